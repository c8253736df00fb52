"""ctypes binding of the tensor-ash C ABI (include/tensor_ash.h).

Loads ``tensor-ash_amd/lib/libtensor_ash.so`` (built by
``tensor-ash_amd/build.py``) and wraps its handles in small Python classes
that follow the reference's Rust API names (``Context``, ``Executor``,
``Tensor``, ``MatmulOp``, ``Epilogue``, ``run_ops``, ``run_op_graph``,
``run_matmuls_split_k2``, ``prepare_ops`` ...).  There is no CPU fallback:
every compute call goes through the HIP library, and a missing library is
an ImportError.
"""

from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

_PKG = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("TA_LIBRARY", _PKG / "lib" / "libtensor_ash.so"))

if not LIB_PATH.exists():
    raise ImportError(f"{LIB_PATH} is missing: build it with `python tensor-ash_amd/build.py`")

_lib = C.CDLL(str(LIB_PATH))

ACTIVATION_NONE, ACTIVATION_RELU, ACTIVATION_SILU, ACTIVATION_GELU = 0, 1, 2, 3
BINARY_NONE, BINARY_ADD_SCALED, BINARY_MUL = 0, 1, 2


class TensorAshError(RuntimeError):
    """A tensor-ash call returned -1 / NULL; the message is ta_last_error()."""


class RunStats(C.Structure):
    _fields_ = [("has_gpu_time", C.c_uint32), ("gpu_time_ns", C.c_uint64), ("n_calls", C.c_size_t),
                ("total_flops", C.c_uint64), ("tflops", C.c_double)]


class _Call(C.Structure):
    _fields_ = [("a", C.c_void_p), ("b", C.c_void_p), ("c", C.c_void_p), ("alpha", C.c_float),
                ("accumulate", C.c_uint32)]


class _Epilogue(C.Structure):
    _fields_ = [("bias", C.c_void_p), ("activation", C.c_uint32), ("binary_kind", C.c_uint32),
                ("d", C.c_void_p), ("beta", C.c_float)]


class _Op(C.Structure):
    _fields_ = [("call", _Call), ("epilogue", _Epilogue)]


class _OpV2(C.Structure):
    _fields_ = [("base", _Op), ("packed_b", C.c_uint32), ("reserved", C.c_uint32 * 3)]


class _StoreDesc(C.Structure):
    _fields_ = [("head_dim", C.c_uint32), ("pos_base", C.c_uint32), ("pos_scale", C.c_uint32),
                ("stride_head", C.c_uint32), ("stride_dim", C.c_uint32), ("reserved", C.c_uint32),
                ("pos_addr", C.c_uint64)]


class _OpV3(C.Structure):
    _fields_ = [("v2", _OpV2), ("norm_weight", C.c_void_p), ("norm_eps", C.c_float),
                ("store_kind", C.c_uint32), ("store_table", C.c_void_p), ("store_dst", C.c_void_p),
                ("store", _StoreDesc)]


class _RopeDesc(C.Structure):
    _fields_ = [("heads", C.c_uint32), ("head_dim", C.c_uint32), ("rot_dim", C.c_uint32), ("pos_base", C.c_uint32)]


class _CopyDesc(C.Structure):
    _fields_ = [("extent", C.c_uint32 * 3), ("src_offset", C.c_uint32), ("src_strides", C.c_uint32 * 3),
                ("dst_offset", C.c_uint32), ("dst_strides", C.c_uint32 * 3)]


class _FlashDesc(C.Structure):
    _fields_ = [("kv_len", C.c_uint32), ("pos_base", C.c_uint32), ("scale", C.c_float),
                ("token_major_heads", C.c_uint32), ("out_token_major_heads", C.c_uint32),
                ("reserved", C.c_uint32)]


class _AttnDecodeDesc(C.Structure):
    _fields_ = [("kv_len", C.c_uint32), ("scale", C.c_float), ("pos_addr", C.c_uint64)]


class _RopeScatterDesc(C.Structure):
    _fields_ = [("dst_offset", C.c_uint32), ("dst_strides", C.c_uint32 * 3), ("pos_scale", C.c_uint32),
                ("reserved", C.c_uint32)]


class _QkvPackDesc(C.Structure):
    _fields_ = [("heads", C.c_uint32), ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("rot_dim", C.c_uint32), ("pos_base", C.c_uint32), ("reserved", C.c_uint32)]


class _ExecOp(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("mask_kind", C.c_uint32), ("valid_or_prefix", C.c_uint32),
                ("rows_per_group", C.c_uint32), ("scalar", C.c_float), ("pos_scale", C.c_uint32),
                ("pos_addr", C.c_uint64), ("inp", C.c_void_p * 3), ("out", C.c_void_p),
                ("matmul", C.POINTER(_OpV3)), ("rope", _RopeDesc), ("copy", _CopyDesc),
                ("flash", _FlashDesc), ("cell", C.c_void_p), ("aux", C.c_void_p),
                ("attn", _AttnDecodeDesc), ("aux2", C.c_void_p), ("scatter", _RopeScatterDesc),
                ("binary_op", C.c_uint32), ("qkv", _QkvPackDesc), ("n_jobs", C.c_uint32)]


class _DispatchInfo(C.Structure):
    _fields_ = [("kernel", C.c_char_p), ("tile", C.c_uint32 * 3), ("has_split_k2", C.c_uint32),
                ("split_k2_splits", C.c_uint32)]


def _sig(name, restype, *argtypes):
    fn = getattr(_lib, name)
    fn.restype = restype
    fn.argtypes = list(argtypes)
    return fn


P = C.c_void_p
u32, u64, sz, f32 = C.c_uint32, C.c_uint64, C.c_size_t, C.c_float
_sig("ta_version", C.c_char_p)
_sig("ta_last_error", C.c_char_p)
_sig("ta_context_create", P, u32, C.c_char_p)
_sig("ta_context_destroy", None, P)
_sig("ta_context_supports_f16", u32, P)
_sig("ta_context_supports_bda", u32, P)
_sig("ta_context_cu_count", u32, P)
_sig("ta_executor_create", P, P, sz, u32, C.c_char_p)
_sig("ta_executor_create_v2", P, P, sz, u32, C.c_char_p, u32)
_sig("ta_executor_destroy", None, P)
for _n in ("ta_tensor_create", "ta_tensor_create_on_executor", "ta_tensor_create_f16",
           "ta_tensor_create_f16_on_executor"):
    _sig(_n, P, P, C.POINTER(u32), sz)
_sig("ta_tensor_destroy", None, P)
_sig("ta_tensor_len", u64, P)
_sig("ta_tensor_size_bytes", u64, P)
_sig("ta_tensor_is_f16", u32, P)
_sig("ta_upload", C.c_int, P, P, C.POINTER(f32), sz)
_sig("ta_upload_f16", C.c_int, P, P, C.POINTER(C.c_uint16), sz)
_sig("ta_download", C.c_int, P, P, C.POINTER(f32), sz)
_sig("ta_matmul", C.c_int, P, P, P, P, f32, u32, C.POINTER(RunStats))
_sig("ta_matmul_batch", C.c_int, P, C.POINTER(_Call), sz, C.POINTER(RunStats))
_sig("ta_run_ops", C.c_int, P, C.POINTER(_Op), sz, C.POINTER(RunStats))
_sig("ta_run_op_graph", C.c_int, P, C.POINTER(_Op), sz, C.POINTER(RunStats))
_sig("ta_run_ops_v2", C.c_int, P, C.POINTER(_OpV2), sz, C.POINTER(RunStats))
_sig("ta_run_op_graph_v2", C.c_int, P, C.POINTER(_OpV2), sz, C.POINTER(RunStats))
_sig("ta_matmul_split_k2", C.c_int, P, P, P, P, f32, u32, C.POINTER(RunStats))
_sig("ta_allocation_count", C.c_uint64)
_sig("ta_run_op_split_k2", C.c_int, P, P, u32, C.POINTER(RunStats))
_sig("ta_matmul_split_k2_noalloc", C.c_int, P, P, P, P, f32, u32, C.POINTER(RunStats))
_sig("ta_prepared_create", P, P, C.POINTER(_Op), sz, u32)
_sig("ta_prepared_create_v2", P, P, C.POINTER(_OpV2), sz, u32)
_sig("ta_run_ops_v3", C.c_int, P, C.POINTER(_OpV3), sz, C.POINTER(RunStats))
_sig("ta_run_op_graph_v3", C.c_int, P, C.POINTER(_OpV3), sz, C.POINTER(RunStats))
_sig("ta_prepared_create_v3", P, P, C.POINTER(_OpV3), sz, u32)
_sig("ta_run_gemv_chain", C.c_int, P, C.POINTER(_OpV3), sz, C.POINTER(RunStats))
_sig("ta_tensor_device_address", u64, P)
_sig("ta_flash_attention", C.c_int, P, P, P, P, P, C.POINTER(_FlashDesc), C.POINTER(RunStats))
_sig("ta_run_exec_ops", C.c_int, P, C.POINTER(_ExecOp), sz, C.POINTER(RunStats))
_sig("ta_u32_cell_create", P, P, u32)
_sig("ta_u32_cell_destroy", None, P)
_sig("ta_u32_cell_write", C.c_int, P, C.POINTER(u32), sz)
_sig("ta_u32_cell_read", C.c_int, P, C.POINTER(u32))
_sig("ta_u32_cell_device_address", u64, P)
_sig("ta_u32_cell_cap", u32, P)
_sig("ta_argmax", C.c_int, P, P, P, C.POINTER(RunStats))
_sig("ta_rope_scatter", C.c_int, P, P, P, P, C.POINTER(_RopeDesc), C.POINTER(_RopeScatterDesc), C.POINTER(RunStats))
_sig("ta_binary", C.c_int, P, P, P, P, u32, f32, C.POINTER(RunStats))
_sig("ta_prefill_qkv_pack", C.c_int, P, P, P, P, P, P, C.POINTER(_QkvPackDesc), C.POINTER(RunStats))
_sig("ta_embed_gather", C.c_int, P, P, P, P, C.POINTER(RunStats))
_sig("ta_attn_decode", C.c_int, P, P, P, P, P, P, C.POINTER(_AttnDecodeDesc), C.POINTER(RunStats))
_sig("ta_prepared_create_exec", P, P, C.POINTER(_ExecOp), sz)
_sig("ta_softmax_rows", C.c_int, P, P, P, f32, u32, u32, u32, C.POINTER(RunStats))
_sig("ta_rms_norm", C.c_int, P, P, P, P, f32, C.POINTER(RunStats))
_sig("ta_layer_norm", C.c_int, P, P, P, P, P, f32, C.POINTER(RunStats))
_sig("ta_rope", C.c_int, P, P, P, P, C.POINTER(_RopeDesc), C.POINTER(RunStats))
_sig("ta_copy_strided", C.c_int, P, P, P, C.POINTER(_CopyDesc), C.POINTER(RunStats))
_sig("ta_prepared_run", C.c_int, P, C.POINTER(RunStats))
_sig("ta_prepared_submit", C.c_int, P)
_sig("ta_prepared_wait", C.c_int, P, C.POINTER(RunStats))
_sig("ta_prepared_destroy", None, P)
_sig("ta_dispatch_info_for", C.c_int, P, u32, u32, u32, u32, u32, C.POINTER(_DispatchInfo))
_sig("ta_tune_shape", C.c_int, P, u32, u32, u32, u32)
_sig("ta_pack_f16w_row_tiles", C.c_int, C.POINTER(f32), sz, sz, sz, C.POINTER(f32))
_sig("ta_f16w_row_tile_n", u32, u32, u32)
_sig("ta_kernel_count", sz)
_sig("ta_kernel_name", C.c_char_p, sz)
_sig("ta_kernel_tile", C.c_int, sz, C.POINTER(u32))

lib = _lib


def last_error() -> str:
    return (_lib.ta_last_error() or b"").decode()


def _check(rc: int) -> None:
    if rc != 0:
        raise TensorAshError(last_error())


def _checkp(ptr):
    if not ptr:
        raise TensorAshError(last_error())
    return ptr


def version() -> str:
    return _lib.ta_version().decode()


def kernel_names() -> list[str]:
    return [_lib.ta_kernel_name(i).decode() for i in range(_lib.ta_kernel_count())]


def f16w_row_tile_n(k: int, n: int) -> int:
    return int(_lib.ta_f16w_row_tile_n(k, n))


def allocation_count() -> int:
    """Device and pinned-host allocations the library has made in this
    process (include/tensor_ash.h ta_allocation_count)."""
    return int(_lib.ta_allocation_count())


def pack_f16w_row_tiles(src: np.ndarray, k: int, n: int, tile_n: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.float32).reshape(-1)
    out = np.empty_like(src)
    _check(_lib.ta_pack_f16w_row_tiles(src.ctypes.data_as(C.POINTER(f32)), k, n, tile_n,
                                       out.ctypes.data_as(C.POINTER(f32))))
    return out


class Context:
    def __init__(self, device_preference: Optional[str] = None, enable_validation: bool = False):
        pref = None if device_preference is None else device_preference.encode()
        self._h = _checkp(_lib.ta_context_create(int(enable_validation), pref))

    @property
    def handle(self):
        return self._h

    @property
    def cu_count(self) -> int:
        return int(_lib.ta_context_cu_count(self._h))

    def close(self):
        if self._h:
            _lib.ta_context_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Tensor:
    def __init__(self, ctx: Context, shape: Sequence[int], f16: bool = False):
        arr = (u32 * len(shape))(*shape)
        fn = _lib.ta_tensor_create_f16 if f16 else _lib.ta_tensor_create
        self._h = _checkp(fn(ctx.handle, arr, len(shape)))
        self._ctx = ctx  # keep the context alive
        self.shape = tuple(int(s) for s in shape)
        self.f16 = f16

    @property
    def handle(self):
        return self._h

    def __len__(self):
        return int(_lib.ta_tensor_len(self._h))

    @property
    def size_bytes(self) -> int:
        return int(_lib.ta_tensor_size_bytes(self._h))

    @property
    def device_address(self) -> int:
        """Device address of the allocation (for MatmulStoreDesc.pos_addr)."""
        return int(_lib.ta_tensor_device_address(self._h))

    def close(self):
        if self._h:
            _lib.ta_tensor_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class Epilogue:
    """src/matmul/api.rs:56-105: +bias -> activation -> binary with D."""
    bias: Optional[Tensor] = None
    activation: int = ACTIVATION_NONE
    binary: int = BINARY_NONE
    d: Optional[Tensor] = None
    beta: float = 0.0


STORE_NONE, STORE_ROPE, STORE_SCATTER, STORE_ROPE_SCATTER = 0, 1, 2, 3


@dataclass
class MatmulStoreDesc:
    """src/matmul/api.rs:117-133.  pos_addr: device address of a u32 cell
    (Tensor.device_address), 0 = none."""
    head_dim: int
    pos_base: int = 0
    pos_scale: int = 0
    stride_head: int = 0
    stride_dim: int = 0
    pos_addr: int = 0


@dataclass
class MatmulStore:
    """src/matmul/api.rs:135-206: kind STORE_ROPE (table), STORE_SCATTER
    (dst) or STORE_ROPE_SCATTER (table, dst)."""
    kind: int
    desc: MatmulStoreDesc
    table: Optional[Tensor] = None
    dst: Optional[Tensor] = None


@dataclass
class MatmulOp:
    """src/matmul/api.rs:213-299: with_packed_b -> packed_b=True,
    with_normed_a(w, eps) -> normed_a=(w, eps), with_store_* -> store."""
    a: Tensor
    b: Tensor
    c: Tensor
    alpha: float = 1.0
    accumulate: bool = False
    epilogue: Epilogue = field(default_factory=Epilogue)
    packed_b: bool = False
    normed_a: Optional[tuple] = None
    store: Optional[MatmulStore] = None

    def _raw(self) -> _Op:
        e = self.epilogue
        return _Op(_Call(self.a.handle, self.b.handle, self.c.handle, self.alpha, int(self.accumulate)),
                   _Epilogue(e.bias.handle if e.bias else None, e.activation, e.binary,
                             e.d.handle if e.d else None, e.beta))

    def _raw_v3(self) -> _OpV3:
        op = _OpV3(_OpV2(self._raw(), int(self.packed_b)))
        if self.normed_a is not None:
            op.norm_weight = self.normed_a[0].handle
            op.norm_eps = float(self.normed_a[1])
        if self.store is not None:
            st, d = self.store, self.store.desc
            op.store_kind = st.kind
            op.store_table = st.table.handle if st.table else None
            op.store_dst = st.dst.handle if st.dst else None
            op.store = _StoreDesc(d.head_dim, d.pos_base, d.pos_scale, d.stride_head, d.stride_dim, 0,
                                  d.pos_addr)
        return op


def _ops_array(ops: Sequence[MatmulOp]):
    """(array, version): the narrowest C struct that carries every op."""
    if any(o.normed_a is not None or o.store is not None for o in ops):
        return (_OpV3 * len(ops))(*[o._raw_v3() for o in ops]), 3
    if any(o.packed_b for o in ops):
        arr = (_OpV2 * len(ops))(*[_OpV2(o._raw(), int(o.packed_b)) for o in ops])
        return arr, 2
    return (_Op * len(ops))(*[o._raw() for o in ops]), 1


SOFTMAX_MASK_FULL, SOFTMAX_MASK_PREFIX, SOFTMAX_MASK_CAUSAL = 0, 1, 2
EXEC_MATMUL, EXEC_RMS_NORM, EXEC_LAYER_NORM, EXEC_SOFTMAX_ROWS, EXEC_ROPE, EXEC_COPY_STRIDED, \
    EXEC_FLASH_ATTENTION, EXEC_ARGMAX, EXEC_EMBED_GATHER, EXEC_ATTN_DECODE, EXEC_ROPE_SCATTER, EXEC_BINARY, \
    EXEC_PREFILL_QKV_PACK, EXEC_GEMV_CHAIN = range(14)
# Binary combine ops (src/executor/elementwise/mod.rs:242-252).
BINARY_OP_ADD_SCALED, BINARY_OP_SILU_MUL = 0, 1
# Chunk bound of decode attention; scratch holds kv_heads * ATTN_DECODE_MAX_CHUNKS
# * group * (dh + 2) f32 (src/executor/elementwise/mod.rs:229-232).
ATTN_DECODE_MAX_CHUNKS = 32


class U32Cell:
    """Host-visible u32 cells (src/executor/cells.rs:10-205): pinned, mapped
    host memory that kernels read and write through `device_address` and the
    host through set / write / read between submissions.  The reference's
    PosBuffer and HostU32Buffer are cells of one value, TokenIdBuffer a
    cell of `cap` values; all start zeroed."""

    def __init__(self, ctx: "Context", cap: int = 1):
        self._h = _checkp(_lib.ta_u32_cell_create(ctx.handle, cap))
        self._ctx = ctx

    @property
    def handle(self):
        return self._h

    @property
    def device_address(self) -> int:
        return int(_lib.ta_u32_cell_device_address(self._h))

    @property
    def cap(self) -> int:
        return int(_lib.ta_u32_cell_cap(self._h))

    def set(self, value: int) -> None:
        self.write([value])

    def write(self, values: Sequence[int]) -> None:
        a = np.ascontiguousarray(values, dtype=np.uint32).reshape(-1)
        _check(_lib.ta_u32_cell_write(self._h, a.ctypes.data_as(C.POINTER(u32)), a.size))

    def read(self) -> int:
        v = u32()
        _check(_lib.ta_u32_cell_read(self._h, C.byref(v)))
        return int(v.value)

    def close(self):
        if self._h:
            _lib.ta_u32_cell_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


PosBuffer = HostU32Buffer = TokenIdBuffer = U32Cell
GEMV_CHAIN_MAX_JOBS = 8


def round_f32_via_f16(x):
    """src/dtype.rs:108-112: f32 -> f16 (RNE) -> f32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def f16w_row_uses_k16(k: int, n: int) -> bool:
    """src/pipeline/routing.rs:10-12 as this build routes it: whether the
    packed decode weights of a [k, n] matrix use 32-column tiles."""
    return f16w_row_tile_n(k, n) == 32


@dataclass
class RopeScatterDesc:
    """src/executor/elementwise/mod.rs:144-159: element (t, h, d) goes to
    dst_offset (+ position * pos_scale in a graph with a position cell) +
    t * dst_strides[0] + h * dst_strides[1] + d * dst_strides[2]."""
    dst_offset: int
    dst_strides: Sequence[int]
    pos_scale: int = 0

    def _raw(self) -> _RopeScatterDesc:
        return _RopeScatterDesc(self.dst_offset, (C.c_uint32 * 3)(*self.dst_strides), self.pos_scale, 0)


@dataclass
class PrefillQkvPackDesc:
    """src/executor/elementwise/mod.rs:186-199."""
    heads: int
    kv_heads: int
    head_dim: int
    rot_dim: int
    pos_base: int = 0

    def _raw(self) -> _QkvPackDesc:
        return _QkvPackDesc(self.heads, self.kv_heads, self.head_dim, self.rot_dim, self.pos_base, 0)


@dataclass
class AttnDecodeDesc:
    """src/executor/elementwise/mod.rs:200-227; pos_addr: device address of a
    u32 cell added to kv_len when the op runs (0 = none)."""
    kv_len: int
    scale: float = 1.0
    pos_addr: int = 0

    def _raw(self) -> _AttnDecodeDesc:
        return _AttnDecodeDesc(self.kv_len, self.scale, self.pos_addr)


@dataclass
class RopeDesc:
    """src/executor/elementwise/mod.rs RopeDesc; pos_addr: device address of
    a u32 position cell added to pos_base when the op runs (graphs only)."""
    heads: int
    head_dim: int
    rot_dim: int
    pos_base: int = 0
    pos_addr: int = 0


@dataclass
class CopyDesc:
    """src/executor/elementwise/mod.rs CopyDesc; pos_addr / pos_scale (graphs
    only): the cell's value times pos_scale is added to dst_offset."""
    extent: Sequence[int]
    src_strides: Sequence[int]
    dst_strides: Sequence[int]
    src_offset: int = 0
    dst_offset: int = 0
    pos_addr: int = 0
    pos_scale: int = 0

    def _raw(self) -> _CopyDesc:
        return _CopyDesc((C.c_uint32 * 3)(*self.extent), self.src_offset, (C.c_uint32 * 3)(*self.src_strides),
                         self.dst_offset, (C.c_uint32 * 3)(*self.dst_strides))


@dataclass
class FlashAttentionDesc:
    """src/executor/elementwise/mod.rs:160-184."""
    kv_len: int
    pos_base: int = 0
    scale: float = 1.0
    token_major_heads: Optional[int] = None
    out_token_major_heads: Optional[int] = None

    def _raw(self) -> _FlashDesc:
        return _FlashDesc(self.kv_len, self.pos_base, self.scale, self.token_major_heads or 0,
                          self.out_token_major_heads or 0, 0)


class ExecOp:
    """One step of a mixed-op graph (src/executor/graph_ops.rs:23-171)."""

    def __init__(self, kind: int, keep=(), **fields):
        self.kind = kind
        self._fields = fields
        self._keep = list(keep)

    def _raw(self) -> _ExecOp:
        r = _ExecOp(kind=self.kind)
        for k, v in self._fields.items():
            if k == "inp":
                for i, t in enumerate(v):
                    r.inp[i] = t.handle if t is not None else None
            elif k == "out":
                r.out = v.handle
            else:
                setattr(r, k, v)
        return r

    @staticmethod
    def matmul(op: "MatmulOp") -> "ExecOp":
        raw = op._raw_v3()
        return ExecOp(EXEC_MATMUL, keep=[op, raw], matmul=C.pointer(raw))

    @staticmethod
    def rms_norm(input, weight, output, eps) -> "ExecOp":
        return ExecOp(EXEC_RMS_NORM, keep=[input, weight, output], inp=[input, weight], out=output, scalar=eps)

    @staticmethod
    def layer_norm(input, weight, bias, output, eps) -> "ExecOp":
        return ExecOp(EXEC_LAYER_NORM, keep=[input, weight, bias, output], inp=[input, weight, bias], out=output,
                      scalar=eps)

    @staticmethod
    def softmax_rows(input, output, scale, mask_kind=SOFTMAX_MASK_FULL, valid_or_prefix=0,
                     rows_per_group=0) -> "ExecOp":
        return ExecOp(EXEC_SOFTMAX_ROWS, keep=[input, output], inp=[input], out=output, scalar=scale,
                      mask_kind=mask_kind, valid_or_prefix=valid_or_prefix, rows_per_group=rows_per_group)

    @staticmethod
    def rope(input, table, output, desc: RopeDesc) -> "ExecOp":
        return ExecOp(EXEC_ROPE, keep=[input, table, output], inp=[input, table], out=output,
                      rope=_RopeDesc(desc.heads, desc.head_dim, desc.rot_dim, desc.pos_base),
                      pos_addr=desc.pos_addr)

    @staticmethod
    def copy_strided(src, dst, desc: CopyDesc) -> "ExecOp":
        return ExecOp(EXEC_COPY_STRIDED, keep=[src, dst], inp=[src], out=dst, copy=desc._raw(),
                      pos_addr=desc.pos_addr, pos_scale=desc.pos_scale)

    @staticmethod
    def flash_attn(q, kt, v, out, desc: FlashAttentionDesc) -> "ExecOp":
        return ExecOp(EXEC_FLASH_ATTENTION, keep=[q, kt, v, out], inp=[q, kt, v], out=out, flash=desc._raw())

    @staticmethod
    def gemv_chain(jobs: Sequence["MatmulOp"]) -> "ExecOp":
        raws = [j._raw_v3() for j in jobs]
        arr = (_OpV3 * len(raws))(*raws)
        return ExecOp(EXEC_GEMV_CHAIN, keep=[list(jobs), raws, arr], matmul=C.cast(arr, C.POINTER(_OpV3)),
                      n_jobs=len(raws))

    @staticmethod
    def rope_scatter(input, table, dst, desc: RopeDesc, scatter: RopeScatterDesc) -> "ExecOp":
        return ExecOp(EXEC_ROPE_SCATTER, keep=[input, table, dst], inp=[input, table], out=dst,
                      rope=_RopeDesc(desc.heads, desc.head_dim, desc.rot_dim, desc.pos_base),
                      pos_addr=desc.pos_addr, scatter=scatter._raw())

    @staticmethod
    def binary(a, b, out, op: int, beta: float = 0.0) -> "ExecOp":
        return ExecOp(EXEC_BINARY, keep=[a, b, out], inp=[a, b], out=out, binary_op=op, scalar=beta)

    @staticmethod
    def prefill_qkv_pack(qkv, table, q, kt, v, desc: PrefillQkvPackDesc) -> "ExecOp":
        return ExecOp(EXEC_PREFILL_QKV_PACK, keep=[qkv, table, q, kt, v], inp=[qkv, table], out=q,
                      aux=kt.handle, aux2=v.handle, qkv=desc._raw())

    @staticmethod
    def argmax(input, result: U32Cell) -> "ExecOp":
        return ExecOp(EXEC_ARGMAX, keep=[input, result], inp=[input], cell=result.handle)

    @staticmethod
    def embed_gather(tokens: U32Cell, table, out) -> "ExecOp":
        """EmbedGather (one id, out [embd]) and EmbedGatherRows (t ids, out [t, embd])."""
        return ExecOp(EXEC_EMBED_GATHER, keep=[tokens, table, out], inp=[table], out=out, cell=tokens.handle)

    embed_gather_rows = embed_gather

    @staticmethod
    def attn_decode(q, kt, v, scratch, out, desc: AttnDecodeDesc) -> "ExecOp":
        return ExecOp(EXEC_ATTN_DECODE, keep=[q, kt, v, scratch, out], inp=[q, kt, v], out=out,
                      aux=scratch.handle, attn=desc._raw())


def _exec_array(ops: Sequence[ExecOp]):
    return (_ExecOp * len(ops))(*[o._raw() for o in ops])


class Prepared:
    def __init__(self, exec_: "Executor", ops: Sequence, as_graph: bool, exec_ops: bool = False):
        if exec_ops:
            arr = _exec_array(ops)
            self._h = _checkp(_lib.ta_prepared_create_exec(exec_.handle, arr, len(ops)))
        else:
            arr, ver = _ops_array(ops)
            fn = {1: _lib.ta_prepared_create, 2: _lib.ta_prepared_create_v2, 3: _lib.ta_prepared_create_v3}[ver]
            self._h = _checkp(fn(exec_.handle, arr, len(ops), int(as_graph)))
        self._keep = (exec_, list(ops))

    def run(self) -> RunStats:
        st = RunStats()
        _check(_lib.ta_prepared_run(self._h, C.byref(st)))
        return st

    def submit(self) -> None:
        _check(_lib.ta_prepared_submit(self._h))

    def wait(self) -> RunStats:
        st = RunStats()
        _check(_lib.ta_prepared_wait(self._h, C.byref(st)))
        return st

    def close(self):
        if self._h:
            _lib.ta_prepared_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Executor:
    def __init__(self, ctx: Context, n_slots: int = 2, max_calls_per_submit: int = 64,
                 kernel_selection: Optional[str] = None, tune: Optional[bool] = None):
        sel = None if kernel_selection is None else kernel_selection.encode()
        if tune is None:
            h = _lib.ta_executor_create(ctx.handle, n_slots, max_calls_per_submit, sel)
        else:
            h = _lib.ta_executor_create_v2(ctx.handle, n_slots, max_calls_per_submit, sel, int(tune))
        self._h = _checkp(h)
        self.ctx = ctx

    @property
    def handle(self):
        return self._h

    def tensor(self, shape: Sequence[int], f16: bool = False) -> Tensor:
        return Tensor(self.ctx, shape, f16)

    def upload(self, t: Tensor, data: np.ndarray) -> None:
        a = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        _check(_lib.ta_upload(self._h, t.handle, a.ctypes.data_as(C.POINTER(f32)), a.size))

    def upload_f16(self, t: Tensor, bits: np.ndarray) -> None:
        a = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
        _check(_lib.ta_upload_f16(self._h, t.handle, a.ctypes.data_as(C.POINTER(C.c_uint16)), a.size))

    def download(self, t: Tensor, n: Optional[int] = None) -> np.ndarray:
        n = len(t) if n is None else n
        out = np.empty(n, dtype=np.float32)
        _check(_lib.ta_download(self._h, t.handle, out.ctypes.data_as(C.POINTER(f32)), n))
        return out.reshape(t.shape) if n == len(t) else out

    def tensor_from(self, data: np.ndarray, f16: bool = False, shape=None) -> Tensor:
        t = self.tensor(shape or data.shape, f16)
        self.upload(t, data)
        return t

    def matmul(self, a: Tensor, b: Tensor, c: Tensor, alpha: float = 1.0, accumulate: bool = False) -> RunStats:
        st = RunStats()
        _check(_lib.ta_matmul(self._h, a.handle, b.handle, c.handle, alpha, int(accumulate), C.byref(st)))
        return st

    def matmul_batch(self, calls: Sequence[tuple]) -> RunStats:
        arr = (_Call * len(calls))(*[_Call(a.handle, b.handle, c.handle, al, int(acc))
                                     for (a, b, c, al, acc) in calls])
        st = RunStats()
        _check(_lib.ta_matmul_batch(self._h, arr, len(calls), C.byref(st)))
        return st

    def run_ops(self, ops: Sequence[MatmulOp]) -> RunStats:
        arr, ver = _ops_array(ops)
        st = RunStats()
        fn = {1: _lib.ta_run_ops, 2: _lib.ta_run_ops_v2, 3: _lib.ta_run_ops_v3}[ver]
        _check(fn(self._h, arr, len(ops), C.byref(st)))
        return st

    def run_op_graph(self, ops: Sequence[MatmulOp]) -> RunStats:
        arr, ver = _ops_array(ops)
        st = RunStats()
        fn = {1: _lib.ta_run_op_graph, 2: _lib.ta_run_op_graph_v2, 3: _lib.ta_run_op_graph_v3}[ver]
        _check(fn(self._h, arr, len(ops), C.byref(st)))
        return st

    # ---- model ops (include/tensor_ash.h ta_softmax_rows ... ta_copy_strided) ----
    def softmax_rows(self, input: Tensor, output: Tensor, scale: float = 1.0, mask_kind: int = 0,
                     valid_or_prefix: int = 0, rows_per_group: int = 0) -> RunStats:
        st = RunStats()
        _check(_lib.ta_softmax_rows(self._h, input.handle, output.handle, scale, mask_kind, valid_or_prefix,
                                    rows_per_group, C.byref(st)))
        return st

    def rms_norm(self, input: Tensor, weight: Tensor, output: Tensor, eps: float) -> RunStats:
        st = RunStats()
        _check(_lib.ta_rms_norm(self._h, input.handle, weight.handle, output.handle, eps, C.byref(st)))
        return st

    def layer_norm(self, input: Tensor, weight: Tensor, bias: Tensor, output: Tensor, eps: float) -> RunStats:
        st = RunStats()
        _check(_lib.ta_layer_norm(self._h, input.handle, weight.handle, bias.handle, output.handle, eps,
                                  C.byref(st)))
        return st

    def rope(self, input: Tensor, table: Tensor, output: Tensor, heads: int, head_dim: int, rot_dim: int,
             pos_base: int = 0) -> RunStats:
        st = RunStats()
        d = _RopeDesc(heads, head_dim, rot_dim, pos_base)
        _check(_lib.ta_rope(self._h, input.handle, table.handle, output.handle, C.byref(d), C.byref(st)))
        return st

    def copy_strided(self, src: Tensor, dst: Tensor, extent, src_strides, dst_strides, src_offset: int = 0,
                     dst_offset: int = 0) -> RunStats:
        st = RunStats()
        d = _CopyDesc((C.c_uint32 * 3)(*extent), src_offset, (C.c_uint32 * 3)(*src_strides), dst_offset,
                      (C.c_uint32 * 3)(*dst_strides))
        _check(_lib.ta_copy_strided(self._h, src.handle, dst.handle, C.byref(d), C.byref(st)))
        return st

    def run_matmuls_split_k2(self, a: Tensor, b: Tensor, c: Tensor, splits: int, alpha: float = 1.0) -> RunStats:
        st = RunStats()
        _check(_lib.ta_matmul_split_k2(self._h, a.handle, b.handle, c.handle, alpha, splits, C.byref(st)))
        return st

    def run_op_split_k2(self, op: MatmulOp, splits: int = 0) -> RunStats:
        """run_matmuls_split_k2 for a whole op: the reduce applies the op's
        fused epilogue once to the fixed-order plane sum (include/tensor_ash.h
        ta_run_op_split_k2)."""
        if op.packed_b or op.normed_a is not None or op.store is not None:
            raise TensorAshError("run_op_split_k2: packed B and decode fusions need a decode GEMV route")
        st = RunStats()
        raw = op._raw()
        _check(_lib.ta_run_op_split_k2(self._h, C.byref(raw), splits, C.byref(st)))
        return st

    def run_matmuls_split_k2_noalloc(self, a: Tensor, b: Tensor, c: Tensor, splits: int,
                                     alpha: float = 1.0) -> RunStats:
        """run_matmuls_split_k2 with the partial planes in the library's fixed
        per-device scratch (no device allocation; raises when they do not fit)."""
        st = RunStats()
        _check(_lib.ta_matmul_split_k2_noalloc(self._h, a.handle, b.handle, c.handle, alpha, splits,
                                               C.byref(st)))
        return st

    def prepare_ops(self, ops: Sequence[MatmulOp]) -> Prepared:
        return Prepared(self, ops, False)

    def prepare_op_graph(self, ops: Sequence[MatmulOp]) -> Prepared:
        return Prepared(self, ops, True)

    def run_gemv_chain(self, jobs: Sequence[MatmulOp]) -> RunStats:
        """gemv_chain.rs:181-193: up to GEMV_CHAIN_MAX_JOBS M = 1 row GEMVs on
        row-major f16 weights, in list order."""
        raws = [j._raw_v3() for j in jobs]
        arr = (_OpV3 * len(raws))(*raws)
        st = RunStats()
        _check(_lib.ta_run_gemv_chain(self._h, arr, len(raws), C.byref(st)))
        return st

    # ---- causal prefill attention and mixed-op graphs ----
    def flash_attention(self, q: Tensor, kt: Tensor, v: Tensor, out: Tensor, desc: FlashAttentionDesc) -> RunStats:
        st = RunStats()
        d = desc._raw()
        _check(_lib.ta_flash_attention(self._h, q.handle, kt.handle, v.handle, out.handle, C.byref(d), C.byref(st)))
        return st

    def rope_scatter(self, input: Tensor, table: Tensor, dst: Tensor, desc: RopeDesc,
                     scatter: RopeScatterDesc) -> RunStats:
        st = RunStats()
        rd, sd = _RopeDesc(desc.heads, desc.head_dim, desc.rot_dim, desc.pos_base), scatter._raw()
        _check(_lib.ta_rope_scatter(self._h, input.handle, table.handle, dst.handle, C.byref(rd), C.byref(sd),
                                    C.byref(st)))
        return st

    def binary(self, a: Tensor, b: Tensor, out: Tensor, op: int, beta: float = 0.0) -> RunStats:
        st = RunStats()
        _check(_lib.ta_binary(self._h, a.handle, b.handle, out.handle, op, beta, C.byref(st)))
        return st

    def prefill_qkv_pack(self, qkv: Tensor, table: Tensor, q: Tensor, kt: Tensor, v: Tensor,
                         desc: PrefillQkvPackDesc) -> RunStats:
        st = RunStats()
        d = desc._raw()
        _check(_lib.ta_prefill_qkv_pack(self._h, qkv.handle, table.handle, q.handle, kt.handle, v.handle,
                                        C.byref(d), C.byref(st)))
        return st

    # ---- the GPU token loop (src/executor/elementwise/ops.rs:456-595, attn.rs) ----
    def create_pos_buffer(self) -> U32Cell:
        return U32Cell(self.ctx, 1)

    def create_host_u32_buffer(self) -> U32Cell:
        return U32Cell(self.ctx, 1)

    def create_token_id_buffer(self, cap: int) -> U32Cell:
        return U32Cell(self.ctx, cap)

    def argmax(self, input: Tensor, result: U32Cell) -> RunStats:
        st = RunStats()
        _check(_lib.ta_argmax(self._h, input.handle, result.handle, C.byref(st)))
        return st

    def embed_gather(self, tokens: U32Cell, table: Tensor, out: Tensor) -> RunStats:
        st = RunStats()
        _check(_lib.ta_embed_gather(self._h, tokens.handle, table.handle, out.handle, C.byref(st)))
        return st

    embed_gather_rows = embed_gather

    def attn_decode(self, q: Tensor, kt: Tensor, v: Tensor, scratch: Tensor, out: Tensor,
                    desc: AttnDecodeDesc) -> RunStats:
        st = RunStats()
        d = desc._raw()
        _check(_lib.ta_attn_decode(self._h, q.handle, kt.handle, v.handle, scratch.handle, out.handle,
                                   C.byref(d), C.byref(st)))
        return st

    def run_exec_ops(self, ops: Sequence[ExecOp]) -> RunStats:
        arr = _exec_array(ops)
        st = RunStats()
        _check(_lib.ta_run_exec_ops(self._h, arr, len(ops), C.byref(st)))
        return st

    def prepare_exec_ops(self, ops: Sequence[ExecOp]) -> Prepared:
        return Prepared(self, ops, True, exec_ops=True)

    def dispatch_info_for(self, batch: int, m: int, n: int, k: int, b_f16: bool = False) -> dict:
        info = _DispatchInfo()
        _check(_lib.ta_dispatch_info_for(self._h, batch, m, n, k, int(b_f16), C.byref(info)))
        return {"kernel": info.kernel.decode(), "tile": tuple(info.tile),
                "split_k2": info.split_k2_splits if info.has_split_k2 else None}

    def tune_shape(self, batch: int, m: int, n: int, k: int) -> None:
        _check(_lib.ta_tune_shape(self._h, batch, m, n, k))

    def close(self):
        if self._h:
            _lib.ta_executor_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
