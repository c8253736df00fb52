"""A C99 program compiled against include/tensor_ash.h and linked to
libtensor_ash.so (tests/c_abi/c_caller.c).  Its _Static_asserts pin the
reference structs' layouts (ref include/tensor_ash.h:16-104); its layout
report must match the ctypes mirror field by field; on the GPU it runs the
reference example's cases (examples/c_smoke.c:55-104)."""

import ctypes as C
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "tests" / "c_abi" / "c_caller.c"
LIB = ROOT / "tensor-ash_amd" / "lib"

MIRROR = {  # header struct -> ctypes class name in tensor_ash
    "ta_run_stats": "RunStats", "ta_matmul_call": "_Call", "ta_epilogue": "_Epilogue",
    "ta_matmul_op": "_Op", "ta_rope_desc": "_RopeDesc", "ta_copy_desc": "_CopyDesc",
    "ta_dispatch_info": "_DispatchInfo", "ta_matmul_op_v2": "_OpV2", "ta_store_desc": "_StoreDesc",
    "ta_matmul_op_v3": "_OpV3", "ta_flash_desc": "_FlashDesc", "ta_rope_scatter_desc": "_RopeScatterDesc",
    "ta_prefill_qkv_pack_desc": "_QkvPackDesc", "ta_attn_decode_desc": "_AttnDecodeDesc",
    "ta_exec_op": "_ExecOp",
}
RENAMED = {("ta_exec_op", "in"): "inp"}  # `in` is a Python keyword


@pytest.fixture(scope="module")
def c_caller(tmp_path_factory):
    cc = shutil.which("cc") or shutil.which("gcc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = tmp_path_factory.mktemp("c_caller") / "c_caller"
    subprocess.run([cc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", str(SRC), "-o", str(exe),
                    f"-L{LIB}", f"-Wl,-rpath,{LIB}", "-ltensor_ash", "-lm"], check=True,
                   capture_output=True, text=True)
    return exe


def test_layout_matches_ctypes_mirror(ta, c_caller):
    out = subprocess.run([str(c_caller), "layout"], check=True, capture_output=True, text=True).stdout
    seen = set()
    for line in out.splitlines():
        parts = line.split()
        cls = getattr(ta, MIRROR[parts[0]])
        seen.add(parts[0])
        if parts[1] == "sizeof":
            assert C.sizeof(cls) == int(parts[2]), line
            continue
        field = getattr(cls, RENAMED.get((parts[0], parts[1]), parts[1]))
        assert (field.offset, field.size) == (int(parts[2]), int(parts[3])), line
    assert seen == set(MIRROR)


@pytest.mark.gpu
def test_c_caller_runs_reference_example_cases(c_caller):
    print("c_caller run", flush=True)
    proc = subprocess.run([str(c_caller), "run"], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr + proc.stdout
    assert "plain 58 64 139 154 flops 24" in proc.stdout
    assert proc.stdout.rstrip().endswith("OK")
