"""Build recipe for the MI355X extension (no torch cpp_extension, no hipify).

Produces, in-tree:
  silvertorch_amd/libsilvertorch_hip.so  HIP kernels + the C ABI
                                         (include/silvertorch_hip.h), gfx950
  silvertorch_amd/_C.so                  torch.ops.st.* registration, linked
                                         against the library above

Run ``python -m silvertorch_amd._build`` or call :func:`build`.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libsilvertorch_hip.so"
EXT = PKG / "_C.so"
# Measurement probe (bench.py --probe-pattern): the search kernel's memory
# access pattern without its evaluation; not part of the product library.
PROBE = PKG / "libst_probe.so"

ARCH = os.environ.get("ST_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed FP32 instructions are disabled for all device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# (source, ST_SEARCH_K) pairs: the search kernel is compiled once per K.
LIB_SOURCES = [
    "st_runtime.hip",
    "bloom_search.hip",
    *[("bloom_search_k.hip", k) for k in range(1, 11)],
    "bloom_build.hip",
    "bloom_compact.hip",
    "bloom_partial.hip",
    "bloom_generic.hip",
    "filtered_topk.hip",
    "kmean_ann.hip",
    "fresh_topk.hip",
    "search_plan.cpp",
    "host_pool.cpp",
    "expression_parser.cpp",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + proc.stdout)
        raise RuntimeError(f"build step failed: {cmd[0]} ... {cmd[-1]}")
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l and "warning: feature flag" not in l)
    if out.strip() and os.environ.get("ST_BUILD_VERBOSE"):
        sys.stderr.write(out + "\n")


def _stale(obj: Path, src: Path) -> bool:
    """True when obj is missing or older than its source or any header."""
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    deps = [src, *CSRC.glob("*.hpp"), ROOT / "include" / "silvertorch_hip.h"]
    return any(d.stat().st_mtime > t for d in deps)


INCREMENTAL = False  # set by `python -m silvertorch_amd._build --incremental`


def _compile_lib_object(spec) -> Path:
    src, k = spec if isinstance(spec, tuple) else (spec, None)
    obj = OBJ / (src + ("" if k is None else f".k{k}") + ".o")
    path = CSRC / src
    if INCREMENTAL and not _stale(obj, path):
        return obj
    if src.endswith(".cpp"):  # host-only C++
        cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-c"]
    else:
        cmd = [HIPCC, *HIP_FLAGS, "-c"]
    if k is not None:
        cmd.append(f"-DST_SEARCH_K={k}")
    cmd += [str(path), "-o", str(obj)]
    _run(cmd)
    return obj


def _torch_paths() -> tuple[list[str], list[str]]:
    import torch

    tdir = Path(torch.__file__).resolve().parent
    inc = [str(tdir / "include"), str(tdir / "include" / "torch" / "csrc" / "api" / "include")]
    libdir = str(tdir / "lib")
    return inc, [libdir]


def build_library(jobs: int = os.cpu_count() or 8) -> Path:
    OBJ.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile_lib_object, LIB_SOURCES))
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
          "-o", str(LIB) + ".tmp"])
    os.replace(str(LIB) + ".tmp", LIB)
    return LIB


def build_extension() -> Path:
    import torch

    inc, libdirs = _torch_paths()
    py_inc = sysconfig.get_paths()["include"]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *[f"-I{p}" for p in inc], f"-I{py_inc}", "-I/opt/rocm/include",
        str(CSRC / "torch_ops.cpp"),
        f"-L{PKG}", "-lsilvertorch_hip",
        *[f"-L{d}" for d in libdirs], "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lc10", "-lc10_hip",
        "-L/opt/rocm/lib", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{d}" for d in libdirs],
        "-o", str(EXT) + ".tmp",
    ]
    _run(cmd)
    os.replace(str(EXT) + ".tmp", EXT)
    return EXT


def build_probe() -> Path:
    _run([HIPCC, *HIP_FLAGS, "-shared", str(CSRC / "pattern_probe.hip"), "-o", str(PROBE) + ".tmp"])
    os.replace(str(PROBE) + ".tmp", PROBE)
    return PROBE


def build(jobs: int = os.cpu_count() or 8) -> None:
    build_library(jobs)
    build_extension()
    build_probe()


if __name__ == "__main__":
    INCREMENTAL = "--incremental" in sys.argv[1:]
    build()
    print(f"built {LIB.relative_to(ROOT)}, {EXT.relative_to(ROOT)} and {PROBE.relative_to(ROOT)}")
