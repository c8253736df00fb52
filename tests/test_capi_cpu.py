"""C-ABI checks that need no GPU (capi/src/api.rs:43-183 null-handle tests):
the library loads, exports every symbol include/tensor_ash.h declares, and
its argument-validation paths report the reference's error text."""

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

HEADER = Path(__file__).resolve().parent.parent / "include" / "tensor_ash.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ta_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(ta):
    names = declared_functions()
    assert len(names) >= 35 + 10
    missing = [n for n in names if not hasattr(ta.lib, n)]
    assert not missing, missing


def test_version(ta):
    assert ta.version().startswith("2.0.0")


def last(ta):
    return ta.last_error()


def test_null_op_entry_points(ta):
    L = ta.lib
    assert L.ta_run_ops(None, None, 0, None) == -1 and "ta_run_ops: exec is null" in last(ta)
    assert L.ta_run_op_graph(None, None, 0, None) == -1 and "ta_run_op_graph: exec is null" in last(ta)
    assert L.ta_run_ops_v2(None, None, 0, None) == -1 and "ta_run_ops_v2: exec is null" in last(ta)
    assert not L.ta_prepared_create(None, None, 0, 0) and "ta_prepared_create: exec is null" in last(ta)
    assert L.ta_prepared_run(None, None) == -1 and "ta_prepared_run: prepared is null" in last(ta)
    assert L.ta_prepared_submit(None) == -1 and "ta_prepared_submit: prepared is null" in last(ta)
    assert L.ta_prepared_wait(None, None) == -1 and "ta_prepared_wait: prepared is null" in last(ta)
    assert L.ta_upload(None, None, None, 0) == -1 and "exec is null" in last(ta)
    assert L.ta_download(None, None, None, 0) == -1 and "ta_download: exec is null" in last(ta)
    assert L.ta_matmul(None, None, None, None, 1.0, 0, None) == -1 and "ta_matmul: exec is null" in last(ta)
    assert L.ta_matmul_split_k2(None, None, None, None, 1.0, 4, None) == -1
    assert "ta_matmul_split_k2: exec is null" in last(ta)
    assert L.ta_matmul_split_k2_noalloc(None, None, None, None, 1.0, 4, None) == -1
    assert "ta_matmul_split_k2_noalloc: exec is null" in last(ta)


def test_null_elementwise_and_diagnostics(ta):
    L = ta.lib
    for fn, args in [("ta_softmax_rows", (None, None, None, 1.0, 0, 0, 0, None)),
                     ("ta_rms_norm", (None, None, None, None, 1e-5, None)),
                     ("ta_layer_norm", (None, None, None, None, None, 1e-5, None)),
                     ("ta_rope", (None, None, None, None, None, None)),
                     ("ta_copy_strided", (None, None, None, None, None))]:
        f = getattr(L, fn)
        if fn in ("ta_softmax_rows", "ta_rms_norm", "ta_layer_norm"):
            f.argtypes = [C.c_void_p] * 3 + ([C.c_float, C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p]
                                             if fn == "ta_softmax_rows" else
                                             [C.c_void_p, C.c_float, C.c_void_p] if fn == "ta_rms_norm" else
                                             [C.c_void_p, C.c_void_p, C.c_float, C.c_void_p])
        assert f(*args) == -1
        assert f"{fn}: exec is null" in last(ta)
    assert L.ta_dispatch_info_for(None, 1, 1, 1, 1, 0, None) == -1
    assert "ta_dispatch_info_for: exec is null" in last(ta)
    assert L.ta_tune_shape(None, 1, 64, 64, 64) == -1 and "ta_tune_shape: exec is null" in last(ta)


def test_destroy_null_and_capabilities(ta):
    L = ta.lib
    L.ta_context_destroy(None)
    L.ta_executor_destroy(None)
    L.ta_tensor_destroy(None)
    L.ta_prepared_destroy(None)
    assert L.ta_context_supports_f16(None) == 0 and L.ta_context_supports_bda(None) == 0
    assert L.ta_tensor_is_f16(None) == 0 and L.ta_tensor_len(None) == 0 and L.ta_tensor_size_bytes(None) == 0
    assert L.ta_context_cu_count(None) == 0
    assert not L.ta_executor_create(None, 2, 8, None) and "ta_executor_create: ctx is null" in last(ta)
    assert not L.ta_tensor_create(None, None, 0) and "ta_tensor_create: ctx is null" in last(ta)


def test_error_is_cleared_by_next_call(ta):
    L = ta.lib
    assert L.ta_run_ops(None, None, 0, None) == -1 and last(ta)
    assert L.ta_pack_f16w_row_tiles(np.zeros(4, np.float32).ctypes.data_as(C.POINTER(C.c_float)), 2, 2, 2,
                                    np.zeros(4, np.float32).ctypes.data_as(C.POINTER(C.c_float))) == 0
    assert last(ta) == ""


def test_context_without_gpu_reports_error(ta):
    try:
        ctx = ta.Context()
    except ta.TensorAshError as e:
        assert "no HIP device" in str(e)
    else:
        ctx.close()
        pytest.skip("a GPU is visible; the no-device path is not reachable")


def test_pack_and_tile(ta, oracle):
    w = np.arange(4 * 4, dtype=np.float32)
    assert ta.pack_f16w_row_tiles(w, 4, 4, 2).tolist() == [0, 1, 4, 5, 8, 9, 12, 13, 2, 3, 6, 7, 10, 11, 14, 15]
    w = np.random.default_rng(0).standard_normal(300 * 192).astype(np.float32)
    assert np.array_equal(ta.pack_f16w_row_tiles(w, 300, 192, 64), oracle.pack_row_tiles(w, 300, 192, 64))
    with pytest.raises(ta.TensorAshError, match="not a multiple of tile_n"):
        ta.pack_f16w_row_tiles(w, 300, 192, 50)
    assert ta.f16w_row_tile_n(2048, 5632) == 64 and ta.f16w_row_tile_n(2048, 96) == 32


def test_registry_names(ta):
    names = ta.kernel_names()
    assert len(names) == len(set(names)) and len(names) == ta.lib.ta_kernel_count()
    assert ta.lib.ta_kernel_name(len(names)) is None
    tile = (C.c_uint32 * 3)()
    assert ta.lib.ta_kernel_tile(0, tile) == 0 and tile[0] == 256 and tile[1] == 256


def test_cpp_mirror_unit_tests(tmp_path):
    """C++ unit tests of the host runtime (resolution, registry, routing,
    split-K planning, tuner helpers, tune store), compiled against the
    built library: the counterpart of the reference's `cargo test` units."""
    import subprocess
    root = Path(__file__).resolve().parent.parent
    exe = tmp_path / "host_tests"
    lib = root / "tensor-ash_amd" / "lib"
    cmd = ["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           str(root / "tests" / "cpp" / "host_tests.cpp"), "-o", str(exe), f"-L{lib}", "-ltensor_ash",
           f"-Wl,-rpath,{lib}", "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib", "-lamdhip64"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all passed" in r.stdout
