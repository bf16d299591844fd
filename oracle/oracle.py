"""Python access to the CPU checkers -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of bench.py import this module.
It is the checker of the HIP path, never part of it.

* :func:`definition` -- ctypes wrapper of ``fwo_definition`` (reference_impl.py:11-35 restated).
* :func:`single_pass` -- ctypes wrapper of ``fwo_single_pass`` (src/cpu/fw_cpu.cpp:340-390 restated).
* :func:`load_ref` -- the reference's own CPU extension compiled into ``oracle/_ref`` (or None).
"""
import ctypes
import importlib.util
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "libfwl_oracle.so")
        if not os.path.isfile(path):
            raise RuntimeError("oracle/libfwl_oracle.so is not built: run python oracle/build_oracle.py")
        lib = ctypes.CDLL(path)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        lib.fwo_definition.argtypes = [P, P, I64, I64, ctypes.c_double, P, P, P, P, P, P, P, ctypes.c_int]
        lib.fwo_definition.restype = ctypes.c_int
        lib.fwo_single_pass.argtypes = [P, P, I64, I64, ctypes.c_double, P, P, P, ctypes.c_int, I64, I64]
        lib.fwo_single_pass.restype = I64
        lib.fwo_round_down.argtypes = [ctypes.c_double]
        lib.fwo_round_down.restype = ctypes.c_float
        _LIB = lib
    return _LIB


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _prep(z, y):
    z = np.ascontiguousarray(z, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.int64)
    assert z.ndim == 2 and y.shape == (z.shape[0],)
    return z, y


def definition(z, y, scale=None, grad=True, nthreads=None):
    """Definition oracle.  Returns dict(H, tau, loss64, loss, kappa, grad, flags, mean)."""
    z, y = _prep(z, y)
    N, C = z.shape
    if scale is None:
        scale = 1.0 / N if N else 1.0
    out = dict(H=np.empty(N, np.float32), tau=np.empty(N, np.float64), loss64=np.empty(N, np.float64),
               loss=np.empty(N, np.float32), kappa=np.empty(N, np.int32), flags=np.empty(N, np.int32),
               grad=np.empty((N, C), np.float32) if grad else None)
    nt = nthreads or min(8, os.cpu_count() or 1)
    rc = _lib().fwo_definition(_ptr(z), _ptr(y), N, C, float(scale), _ptr(out["H"]), _ptr(out["tau"]),
                               _ptr(out["loss64"]), _ptr(out["loss"]), _ptr(out["kappa"]), _ptr(out["grad"]),
                               _ptr(out["flags"]), nt)
    if rc != 0:
        raise ValueError(f"fwo_definition failed ({rc}): C must be >= 1 and targets in [0, C)")
    out["mean"] = np.float32(out["loss"].astype(np.float64).mean()) if N else np.float32(np.nan)
    return out


def single_pass(z, y, scale=None, grad=True, nthreads=None, chunk=0, cap_factor=-1):
    """Streaming restatement.  Returns dict(loss64, kappa, grad, fallbacks)."""
    z, y = _prep(z, y)
    N, C = z.shape
    if scale is None:
        scale = 1.0 / N if N else 1.0
    out = dict(loss64=np.empty(N, np.float64), kappa=np.empty(N, np.int64),
               grad=np.empty((N, C), np.float32) if grad else None)
    nt = nthreads or min(8, os.cpu_count() or 1)
    fb = _lib().fwo_single_pass(_ptr(z), _ptr(y), N, C, float(scale), _ptr(out["loss64"]), _ptr(out["kappa"]),
                                _ptr(out["grad"]), nt, int(chunk), int(cap_factor))
    if fb < 0:
        raise ValueError("fwo_single_pass failed")
    out["fallbacks"] = int(fb)
    return out


def definition_f64(z, y, scale=None):
    """Definition oracle for float64 logits (numpy, fp64): per row sort descending, cumulative sums
    in row order, tau = max_k (S_k - 1)/k (first maximiser; reference_impl.py:15-24), clamped below
    the row maximum; kappa = |{z > tau}|, loss = (1 - z_y) + tau, grad = scale * ([z > tau] / kappa
    - e_y) (fw_cpu.cpp:601-614; float64 logits run through fw_cpu.cpp:697-703).  Rows need a finite
    maximum and targets in [0, C).  Returns dict(tau, loss, kappa, grad, mean)."""
    z = np.ascontiguousarray(z, dtype=np.float64)
    y = np.ascontiguousarray(y, dtype=np.int64)
    N, C = z.shape
    if scale is None:
        scale = 1.0 / N if N else 1.0
    v = -np.sort(-z, axis=1)
    S = np.cumsum(v, axis=1)
    f = (S - 1.0) / np.arange(1, C + 1, dtype=np.float64)
    tau = f[np.arange(N), np.argmax(f, axis=1)] if N else np.zeros(0)
    m = v[:, 0] if N else np.zeros(0)
    hi = (tau >= m) & np.isfinite(m)
    tau = np.where(hi, np.nextafter(m, -np.inf), tau)
    sup = z > tau[:, None]
    kappa = sup.sum(axis=1).astype(np.int32)
    zy = z[np.arange(N), y]
    loss = (1.0 - zy) + tau
    inv = scale / kappa.astype(np.float64)
    grad = np.where(sup, inv[:, None], 0.0)
    grad[np.arange(N), y] -= scale
    return dict(tau=tau, loss=loss, kappa=kappa, grad=grad, mean=loss.mean() if N else np.nan)


def round_down(t):
    return np.float32(_lib().fwo_round_down(float(t)))


def _cpu_flags():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def ref_variant():
    flags = _cpu_flags()
    if {"avx512f", "avx512dq", "avx512bw", "avx512vl", "avx512cd"} <= flags:
        return "avx512"
    if {"avx2", "fma", "bmi2"} <= flags:
        return "avx2"
    return None


def load_ref():
    """Import the compiled reference CPU extension from oracle/_ref, or return None if absent."""
    v = ref_variant()
    if v is None:
        return None
    name = "fw_cpu_ref_" + v
    path = os.path.join(HERE, "_ref", name + ".so")
    if not os.path.isfile(path):
        return None
    import torch  # noqa: F401  (the extension links against torch)
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod
