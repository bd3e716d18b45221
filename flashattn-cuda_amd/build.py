"""In-tree build of the HIP library and its torch binding.

* ``libfa_mi355x.so``: the gfx950 kernels and the C ABI (include/fa_mi355x.h,
  include/fa_probe.h), compiled with hipcc.
* ``_fa_torch<EXT_SUFFIX>``: the torch-extension surface (forward,
  forward_only, decode_paged, ...), plain C++ compiled with g++ against the
  torch headers and linked to ``libfa_mi355x.so``.

Run ``python flashattn-cuda_amd/build.py`` (or ``__graft_entry__.build()``).
Both outputs land next to this file; they are git-ignored but travel with the
tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys
import sysconfig

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = ROOT / "include"
OBJ = HERE / "_build"
LIB_NAME = "libfa_mi355x.so"
EXT_NAME = "_fa_torch"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_SOURCES = ["fa_fwd.hip", "fa_bwd.hip", "fa_decode.hip", "fa_pages.hip", "fa_probe.hip"]
CPP_SOURCES = ["fa_capi.cpp"]

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Packed FP32 VALU ops stay off: ordinary float code only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: the softmax reads S directly and O
    # is never copied through AGPRs.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def lib_path() -> pathlib.Path:
    return HERE / LIB_NAME


def ext_path() -> pathlib.Path:
    return HERE / (EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in r.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in line)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(map(str, cmd))}\n{out}")
    return out


def build_lib(jobs: int = 4, extra_flags=()) -> pathlib.Path:
    """Compile every HIP/C++ source for gfx950 and link libfa_mi355x.so."""
    OBJ.mkdir(exist_ok=True)
    cmds, objs = [], []
    for src in HIP_SOURCES:
        obj = OBJ / (src + ".o")
        cmds.append([HIPCC, *HIP_FLAGS, *extra_flags, "-c", "-x", "hip", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    for src in CPP_SOURCES:
        obj = OBJ / (src + ".o")
        cmds.append([HIPCC, "-O2", "-std=c++17", "-fPIC", f"-I{INCLUDE}", "-c", str(CSRC / src),
                     "-o", str(obj)])
        objs.append(obj)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for out in ex.map(_run, cmds):
            if out.strip():
                print(out)
    tmp = OBJ / (LIB_NAME + ".tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, lib_path())
    return lib_path()


def _torch_flags():
    import torch
    from torch.utils import cpp_extension as ce

    inc = [f"-I{p}" for p in ce.include_paths()]
    inc += [f"-I{sysconfig.get_paths()['include']}", "-I/opt/rocm/include", f"-I{INCLUDE}"]
    defs = [
        f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
    ]
    libdirs = ce.library_paths()
    libs = [f"-L{d}" for d in libdirs] + ["-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
                                         "-ltorch_hip", "-ltorch_python"]
    rpath = [f"-Wl,-rpath,{d}" for d in libdirs] + ["-Wl,-rpath,$ORIGIN"]
    return inc, defs, libs, rpath


def build_ext() -> pathlib.Path:
    """Compile the torch binding (g++) and link it to libfa_mi355x.so."""
    inc, defs, libs, rpath = _torch_flags()
    cxx = shutil.which("g++") or "g++"
    tmp = OBJ / (EXT_NAME + ".so.tmp")
    OBJ.mkdir(exist_ok=True)
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", *defs, *inc,
          str(CSRC / "torch_binding.cpp"), "-o", str(tmp),
          f"-L{HERE}", "-l:" + LIB_NAME, *libs, *rpath])
    os.replace(tmp, ext_path())
    return ext_path()


def build_all(jobs: int = 4) -> None:
    build_lib(jobs=jobs)
    build_ext()


if __name__ == "__main__":
    build_all(jobs=int(os.environ.get("MAX_JOBS", "4")))
    print(lib_path())
    print(ext_path())
    sys.exit(0)
