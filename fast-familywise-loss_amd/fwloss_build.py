"""Build driver for the native parts of the package (in-tree, no JIT cache).

* ``libfwloss.so``      -- HIP kernels + C ABI (csrc/*.hip, include/fwloss.h), hipcc for gfx950.
* ``fw_radix_cuda*.so`` -- the PyTorch extension (csrc/fw_radix_ext.cpp), host C++ only, linked
                          against libfwloss.so with an $ORIGIN rpath.

``python fwloss_build.py`` builds both.
"""
import os
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libfwloss.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",   # loadable by the HIP runtime bundled with torch
    # no packed-FP32 instructions (build notes)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-flax-vector-conversions=none",   # no implicit reinterpretation between vector types
]


def _run(cmd):
    print("+ " + " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def ext_path():
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return os.path.join(PKG, "fw_radix_cuda" + suffix)


HIP_SOURCES = ["fwloss.hip", "fwl_f64.hip", "fwl_linear.hip"]   # share csrc/fwl_common.h


def build_lib():
    """Compile every HIP source to an object (in parallel), then link libfwloss.so."""
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    objs, procs = [], []
    for src in HIP_SOURCES:
        obj = os.path.join(CSRC, src.replace(".hip", ".o"))
        cmd = [hipcc] + HIP_FLAGS + ["-c", f"-I{INCLUDE}", os.path.join(CSRC, src), "-o", obj]
        print("+ " + " ".join(cmd), flush=True)
        procs.append(subprocess.Popen(cmd))
        objs.append(obj)
    failed = [src for src, p in zip(HIP_SOURCES, procs) if p.wait() != 0]
    if failed:
        raise subprocess.CalledProcessError(1, f"hipcc {' '.join(failed)}")
    tmp = LIB + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC"] + objs + ["-o", tmp])
    os.replace(tmp, LIB)
    for obj in objs:
        os.remove(obj)
    return LIB


def build_ext():
    import torch
    from torch.utils import cpp_extension as ce
    out = ext_path()
    tmp = out + ".tmp"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = [f"-I{INCLUDE}"]
    for p in ce.include_paths() + [sysconfig.get_paths()["include"], os.path.join(ROCM, "include")]:
        inc += ["-isystem", p]
    libdir = ce.library_paths()[0]
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-parameter",
          "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=fw_radix_cuda",
          "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}"] + inc +
         [os.path.join(CSRC, "fw_radix_ext.cpp"), "-o", tmp, f"-L{PKG}", "-lfwloss",
          f"-L{libdir}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}"])
    os.replace(tmp, out)
    return out


def build_all():
    build_lib()
    build_ext()


if __name__ == "__main__":
    if "--lib" in sys.argv:
        build_lib()
    else:
        build_all()
