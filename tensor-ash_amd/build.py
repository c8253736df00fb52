"""Build the gfx950 code objects, the C-ABI library and the CPU oracle.

Role of the reference's build.rs (glslc -> SPIR-V, build.rs:9-64): every
kernels/*.hip becomes lib/kernels/<name>.hsaco via `hipcc --genco
--offload-arch=gfx950`, loaded at run time with hipModuleLoadData; the C++
host runtime becomes lib/libtensor_ash.so (exports include/tensor_ash.h).
oracle/oracle.c becomes oracle/liboracle.so (test infrastructure only).

    python tensor-ash_amd/build.py            # build everything
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")

# No packed-FP32 instructions anywhere in the device code.
HIP_FLAGS = [
    "--genco",
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
HOST_FLAGS = [
    "-O2", "-g", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
    "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}")


def build_kernels(jobs: int = 4) -> list[Path]:
    out_dir = LIB / "kernels"
    out_dir.mkdir(parents=True, exist_ok=True)
    for stale in out_dir.glob("*.hsaco"):
        stale.unlink()
    srcs = sorted((CSRC / "kernels").glob("*.hip"))
    outs = [out_dir / (s.stem + ".hsaco") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = [pool.submit(_run, [HIPCC, *HIP_FLAGS, str(s), "-o", str(o)]) for s, o in zip(srcs, outs)]
        for f in futs:
            f.result()
    return outs


def build_host(jobs: int = 4) -> Path:
    obj_dir = PKG / "_build"
    obj_dir.mkdir(exist_ok=True)
    srcs = sorted((CSRC / "runtime").glob("*.cpp"))
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    cxx = shutil.which("g++") or "g++"
    # runtime/*.hip hold device data of the library itself (the fixed
    # scratch array): compiled by hipcc into objects with an embedded
    # gfx950 fat binary, linked like the host objects.
    dev_srcs = sorted((CSRC / "runtime").glob("*.hip"))
    dev_objs = [obj_dir / (s.stem + ".hip.o") for s in dev_srcs]
    dev_flags = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
                 "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = [pool.submit(_run, [cxx, *HOST_FLAGS, "-c", str(s), "-o", str(o)]) for s, o in zip(srcs, objs)]
        futs += [pool.submit(_run, [HIPCC, *dev_flags, "-c", str(s), "-o", str(o)])
                 for s, o in zip(dev_srcs, dev_objs)]
        for f in futs:
            f.result()
    objs += dev_objs
    LIB.mkdir(exist_ok=True)
    so = LIB / "libtensor_ash.so"
    _run([cxx, "-shared", "-o", str(so), *map(str, objs), f"-L{ROCM / 'lib'}",
          f"-Wl,-rpath,{ROCM / 'lib'}", "-lamdhip64", "-ldl", "-Wl,--no-undefined"])
    return so


def build_oracle() -> Path:
    src = ROOT / "oracle" / "oracle.c"
    so = ROOT / "oracle" / "liboracle.so"
    gcc = shutil.which("gcc") or "gcc"
    _run([gcc, "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-fPIC", "-shared",
          str(src), "-o", str(so), "-lm"])
    return so


def build_vendor_bench() -> Path:
    """lib/vendor_bench: the hipBLASLt FP32 SGEMM timing binary (comparison
    baseline, not part of the library)."""
    src = PKG / "vendor_bench" / "vendor_bench.cpp"
    out = LIB / "vendor_bench"
    LIB.mkdir(exist_ok=True)
    cxx = shutil.which("g++") or "g++"
    _run([cxx, "-O2", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", str(src),
          "-o", str(out), f"-L{ROCM / 'lib'}", f"-Wl,-rpath,{ROCM / 'lib'}", "-lhipblaslt", "-lamdhip64"])
    return out


def build_handoff_probe() -> Path:
    """lib/handoff_probe: the cross-workgroup hand-off latency probe
    (measurement tool, not part of the library)."""
    src = PKG / "vendor_bench" / "handoff_probe.cpp"
    out = LIB / "handoff_probe"
    LIB.mkdir(exist_ok=True)
    _run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
          "-packed-fp32-ops", str(src), "-o", str(out)])
    return out


def build_all() -> None:
    with cf.ThreadPoolExecutor(max_workers=4) as pool:
        futs = [pool.submit(build_kernels), pool.submit(build_host), pool.submit(build_oracle),
                pool.submit(build_vendor_bench), pool.submit(build_handoff_probe)]
        for f in futs:
            f.result()


if __name__ == "__main__":
    build_all()
    print("built", LIB / "libtensor_ash.so", file=sys.stderr)
