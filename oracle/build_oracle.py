"""Build recipe for the CPU checkers under oracle/ -- TEST INFRASTRUCTURE ONLY.

* ``libfwl_oracle.so``: the C restatement (fwl_oracle.c), built with gcc.
* ``_ref/fw_cpu_ref_{avx512,avx2}.so``: the reference's own CPU path, compiled from its single
  source file where it lies (``/root/reference/src/cpu/fw_cpu.cpp``) against the installed torch,
  with the flags of the reference's JIT build (src/cpu/fwcpp.py:11-15) except that ``-march=native``
  is replaced by the portable x86-64-v4 / x86-64-v3 levels, because the .so is built here and run on
  another host.  Nothing from the reference is copied into the repository; outputs go to
  ``oracle/_ref/`` only (git-ignored).

Run ``python oracle/build_oracle.py [--ref]``.
"""
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REF_SRC = "/root/reference/src/cpu/fw_cpu.cpp"
REF_VARIANTS = {"avx512": "-march=x86-64-v4", "avx2": "-march=x86-64-v3"}


def _run(cmd):
    print("+ " + " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_oracle():
    out = os.path.join(HERE, "libfwl_oracle.so")
    _run(["gcc", "-O3", "-std=c11", "-Wall", "-Wextra", "-fPIC", "-shared", "-fopenmp",
          "-ffp-contract=off", "-march=x86-64-v2", os.path.join(HERE, "fwl_oracle.c"),
          "-o", out, "-lm"])
    return out


def ref_available():
    return os.path.isfile(REF_SRC)


def _ref_cmd(variant):
    import torch
    from torch.utils import cpp_extension as ce
    name = "fw_cpu_ref_" + variant
    out = os.path.join(HERE, "_ref", name + ".so")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = []
    for p in ce.include_paths() + [sysconfig.get_paths()["include"]]:
        inc += ["-isystem", p]
    libdir = ce.library_paths()[0]
    return out, (["g++", "-O3", "-fopenmp", "-fno-math-errno", REF_VARIANTS[variant], "-std=c++17",
                  "-fPIC", "-shared", "-w", f"-DTORCH_EXTENSION_NAME={name}",
                  "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}"] + inc +
                 [REF_SRC, "-o", out, f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu",
                  "-ltorch_python", f"-Wl,-rpath,{libdir}"])


def build_ref():
    """Compile the reference CPU path into oracle/_ref (only where /root/reference exists)."""
    if not ref_available():
        print("oracle/_ref: reference source absent, skipped", flush=True)
        return []
    os.makedirs(os.path.join(HERE, "_ref"), exist_ok=True)
    cmds = [_ref_cmd(v) for v in REF_VARIANTS]
    with ThreadPoolExecutor(len(cmds)) as ex:
        list(ex.map(lambda oc: _run(oc[1]), cmds))
    return [o for o, _ in cmds]


if __name__ == "__main__":
    build_oracle()
    if "--ref" in sys.argv:
        build_ref()
