"""In-tree build of the gfx950 attention library and its torch binding.

Produces, next to this file under ``lib/``:
  * ``libfa2_mi355x.so``  -- the HIP kernels behind the C ABI of
    ``include/fa2_mi355x.h`` (hipcc, --offload-arch=gfx950);
  * ``_fa2_torch<EXT_SUFFIX>`` -- the thin PyTorch-ROCm extension exposing the
    reference's ``fa_fwd``/``fa_bwd``/``rope_fwd``/``rope_bwd`` ops on top of
    that C ABI (g++, linked with an ``$ORIGIN`` rpath);
  * ``libfa2_clock_probe.so`` -- bench.py's in-process clock reading (a
    one-wave s_memtime / s_memrealtime probe; not part of the C ABI).

Run ``python universal-lm-trainer_amd/build.py`` (or ``__graft_entry__.build()``).
No GPU is needed: hipcc cross-compiles for gfx950.
"""

import concurrent.futures
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
REPO = os.path.dirname(HERE)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["fa2_fwd.hip", "fa2_bwd.hip", "fa2_rope.hip", "fa2_capi.hip"]
LIB_NAME = "libfa2_mi355x.so"
EXT_NAME = "_fa2_torch"

# Packed fp32 VALU ops are switched off for every device compile.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def lib_path():
    return os.path.join(LIB, LIB_NAME)


def ext_path():
    return os.path.join(LIB, EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def build_library(verbose=False):
    os.makedirs(LIB, exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(LIB, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as ex:
        for out in ex.map(_run, cmds):
            if verbose and out.strip():
                print(out)
    tmp = lib_path() + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, lib_path())
    for o in objs:
        os.remove(o)
    return lib_path()


def build_extension(verbose=False):
    import torch  # noqa: F401  (header/library locations)
    from torch.utils import cpp_extension

    inc = cpp_extension.include_paths(device_type="cuda") + [os.path.join(ROCM, "include"),
                                                              sysconfig.get_paths()["include"]]
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    tmp = ext_path() + ".tmp"
    cmd = [
        "g++", "-O2", "-std=c++17", "-shared", "-fPIC",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=" + EXT_NAME,
        "-DTORCH_API_INCLUDE_EXTENSION_H", "-D_GLIBCXX_USE_CXX11_ABI=" + str(int(torch._C._GLIBCXX_USE_CXX11_ABI)),
        *[f"-I{p}" for p in inc],
        os.path.join(CSRC, "torch_binding.cpp"),
        "-o", tmp,
        f"-L{torch_lib}", f"-L{LIB}",
        "-lfa2_mi355x", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
    ]
    out = _run(cmd)
    if verbose and out.strip():
        print(out)
    os.replace(tmp, ext_path())
    return ext_path()


def clock_probe_path():
    return os.path.join(LIB, "libfa2_clock_probe.so")


def build_clock_probe(verbose=False):
    tmp = clock_probe_path() + ".tmp"
    out = _run([HIPCC, *HIP_FLAGS, "-shared", os.path.join(CSRC, "clock_probe.hip"), "-o", tmp])
    if verbose and out.strip():
        print(out)
    os.replace(tmp, clock_probe_path())
    return clock_probe_path()


def build(verbose=False):
    build_library(verbose)
    build_extension(verbose)
    build_clock_probe(verbose)
    return lib_path(), ext_path(), clock_probe_path()


if __name__ == "__main__":
    for p in build(verbose="-v" in sys.argv):
        print("built", p)
