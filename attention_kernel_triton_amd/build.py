"""Build recipe for libakt_amd.so (the gfx950 kernel library).

Compiles every ``csrc/*.hip`` for gfx950 with hipcc and links them into
``attention_kernel_triton_amd/libakt_amd.so``, and compiles the host layer
``csrc/torch_ops.cpp`` into the extension module ``_akt_torch`` (both in-tree,
so the built libraries travel with the source tree).  Run ``python -m attention_kernel_triton_amd.build``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libakt_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# Packed FP32 instructions are switched off for all device code.  The atomic
# optimizer is off: every atomic here is issued by one lane, and the optimizer's
# rewrite of a uniform-address atomic reads the returned value at once, which
# makes the wave wait (vmcnt(0)) for every load it has in flight.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-pass-failed",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
]
# Extra flags of single sources.  prefill_wide.hip holds the head-dim 192 and 256
# prefill instances; LLVM's iterative ILP scheduler runs them 8-12% faster than
# the default scheduler (it is 1-2% slower for the D = 64 instances in prefill.hip).
SOURCE_FLAGS = {
    "prefill_wide.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
}


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: set ROCM_PATH or put hipcc on PATH")
    return found


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that line.
    err = "\n".join(l for l in proc.stderr.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def torch_ext_path() -> Path:
    return PKG_DIR / ("_akt_torch" + sysconfig.get_config_var("EXT_SUFFIX"))


def torch_ext_command(out: Path) -> list[str]:
    """g++ line of the compiled host layer (csrc/torch_ops.cpp -> _akt_torch).

    Host code only, built against torch's headers and libraries.  It is not
    linked to libakt_amd.so: the package loads that library with RTLD_GLOBAL
    first, and the extension's akt_* references resolve against it.
    """
    import torch
    import torch.utils.cpp_extension as ce

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    return [
        "g++", "-O2", "-std=c++17", "-shared", "-fPIC",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        "-DTORCH_EXTENSION_NAME=_akt_torch", "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *[f"-I{p}" for p in ce.include_paths("cuda")],
        f"-I{sysconfig.get_paths()['include']}",
        str(CSRC / "torch_ops.cpp"),
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        "-ltorch_python", f"-Wl,-rpath,{torch_lib}",
        "-o", str(out),
    ]


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile all kernels and the host layer and link the shared libraries;
    returns the kernel library's path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no sources under {CSRC}")
    cc = hipcc()
    objs = []
    cmds = []
    for src in sources:
        obj = BUILD_DIR / (src.stem + ".o")
        objs.append(obj)
        cmds.append([cc, *COMMON_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o",
                     str(obj)])
    ext_out = torch_ext_path()
    ext_tmp = ext_out.with_name(ext_out.name + ".tmp")
    cmds.append(torch_ext_command(ext_tmp))
    jobs = jobs or min(len(cmds), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for cmd, _ in zip(cmds, ex.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(link))
    _run(link)
    os.replace(tmp, LIB_PATH)
    os.replace(ext_tmp, ext_out)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
