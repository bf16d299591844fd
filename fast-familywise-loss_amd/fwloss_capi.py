"""ctypes binding of libfwloss.so's C ABI (include/fwloss.h).

This is the binding a Python caller without the torch extension would use (see INTEGRATION.md for
the same stubs in other languages).  Pointers are passed as integers, so any device allocator
works; the helpers below take torch tensors for convenience.  ``torch`` is imported before the
library is opened so that the process holds a single HIP runtime (torch's).
"""
import ctypes
import os
import re

import torch  # noqa: F401  (must precede loading libfwloss.so)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfwloss.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "fwloss.h")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_D = ctypes.c_double

SIGNATURES = {
    "fwl_status_string": ([ctypes.c_int], ctypes.c_char_p),
    "fwl_workspace_bytes": ([_I64, _I64], ctypes.c_size_t),
    "fwl_workspace_bytes_ex": ([_I64, _I64, _P], ctypes.c_size_t),
    "fwl_noalloc_scratch_bytes": ([], ctypes.c_size_t),
    "fwl_forward_backward_noalloc": ([ctypes.c_int, _P, _I64, _P, _I64, _I64, _D, _D, _P, _P, _P, _P, _P, _P, _P, _P],
                                     ctypes.c_int),
    "fwl_forward_backward_ex": ([ctypes.c_int, _P, _I64, _P, _I64, _I64, _D, _D, _P, _P, _P, _P, _P, _P, _P,
                                 ctypes.c_size_t, _P, _P], ctypes.c_int),
    "fwl_forward_backward": ([_P, _P, _I64, _I64, _D, _D, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P], ctypes.c_int),
    "fwl_forward_small": ([_P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P], ctypes.c_int),
    "fwl_backward_small": ([_P, _P, _P, _I64, _I64, _P, _P], ctypes.c_int),
    "fwl_forward_large": ([_P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P], ctypes.c_int),
    "fwl_backward_large": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _P, _P], ctypes.c_int),
    "fwl_scale_grad": ([_P, _P, _I64, _I64, _I64, _P], ctypes.c_int),
    "fwl_forward_backward_typed": ([ctypes.c_int, _P, _P, _I64, _I64, _D, _D, _P, _P, _P, _P, _P, _P,
                                    ctypes.c_size_t, _P], ctypes.c_int),
    "fwl_scale_grad_typed": ([ctypes.c_int, _P, _P, _I64, _I64, _I64, _P], ctypes.c_int),
    "fwl_set_params": ([ctypes.c_int, ctypes.c_int], ctypes.c_int),
    "fwl_get_params": ([ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "fwl_forward_backward_f64": ([_P, _P, _I64, _I64, _D, _D, _P, _P, _P, _P, _P, _P], ctypes.c_int),
    "fwl_scale_grad_f64": ([_P, _P, _I64, _I64, _I64, _P], ctypes.c_int),
    "fwl_linear_state_bytes": ([_I64], ctypes.c_size_t),
    "fwl_linear_support_cap": ([], ctypes.c_int),
    "fwl_linear_begin": ([_P, _I64, _P], ctypes.c_int),
    "fwl_linear_chunk": ([ctypes.c_int, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P], ctypes.c_int),
    "fwl_linear_finish": ([_P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P], ctypes.c_int),
    "fwl_linear_dhidden": ([ctypes.c_int, _P, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _P, _P], ctypes.c_int),
    "fwl_linear_coo": ([_P, _I64, _I64, _P, _P, _P, _P, _I64, _P, _P, _P], ctypes.c_int),
    "fwl_linear_dweight": ([ctypes.c_int, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _P], ctypes.c_int),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.isfile(LIB_PATH):
            raise RuntimeError("libfwloss.so is not built; run python fast-familywise-loss_amd/fwloss_build.py")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def declared_functions():
    """Names of the functions declared in include/fwloss.h."""
    with open(HEADER_PATH) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(fwl_[a-z0-9_]+)\s*\(", text, re.M)))


def status_string(rc):
    return lib().fwl_status_string(rc).decode()


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check(rc, name):
    if rc != 0:
        raise RuntimeError(f"{name}: {status_string(rc)} ({rc})")


class Options(ctypes.Structure):
    """struct fwl_options: the dispatch switches of one call."""
    _fields_ = [("path", ctypes.c_int), ("cand_cap", ctypes.c_int)]


class Workspace:
    """Device workspace (any contents: the library writes what it reads there first)."""

    def __init__(self, device, nbytes=1 << 16):
        self.buf = torch.empty(nbytes, dtype=torch.uint8, device=device)

    def get(self, N, C, options=None):
        need = lib().fwl_workspace_bytes_ex(N, C, None if options is None else ctypes.byref(options))
        if self.buf.numel() < need:
            self.buf = torch.empty(need, dtype=torch.uint8, device=self.buf.device)
        return self.buf


def forward_backward(z, y, scale=None, reduce_div=None, ws=None, grad=None):
    """Fused op through the C ABI.  Returns dict(H, loss, mean, kappa, grad); `grad` may supply the
    gradient buffer (a contiguous [N, C] float32 tensor, e.g. a view at any offset)."""
    N, C = z.shape
    scale = (1.0 / N if N else 1.0) if scale is None else scale
    reduce_div = float(N) if reduce_div is None else reduce_div
    ws = ws or Workspace(z.device)
    buf = ws.get(N, C)
    if grad is not None and (tuple(grad.shape) != (N, C) or grad.dtype != torch.float32 or not grad.is_contiguous()):
        raise ValueError("grad must be a contiguous float32 [N, C] tensor")
    out = dict(H=torch.empty(N, device=z.device), loss=torch.empty(N, device=z.device),
               mean=torch.empty((), device=z.device), kappa=torch.empty(N, dtype=torch.int32, device=z.device),
               grad=torch.empty_like(z) if grad is None else grad)
    rc = lib().fwl_forward_backward(_ptr(z), _ptr(y), N, C, scale, reduce_div, _ptr(out["H"]), _ptr(out["loss"]),
                                    _ptr(out["mean"]), _ptr(out["kappa"]), _ptr(out["grad"]), _ptr(buf),
                                    buf.numel(), _stream())
    _check(rc, "fwl_forward_backward")
    return out


DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}   # enum fwl_dtype


def forward_backward_typed(z, y, scale=None, reduce_div=None, ws=None, grad=None):
    """fwl_forward_backward_typed for float32/bfloat16/float16 logits; grad has the logits' dtype
    (`grad` may supply it: a contiguous [N, C] tensor of that dtype, e.g. a view at any offset)."""
    N, C = z.shape
    scale = (1.0 / N if N else 1.0) if scale is None else scale
    reduce_div = float(N) if reduce_div is None else reduce_div
    ws = ws or Workspace(z.device)
    buf = ws.get(N, C)
    if grad is not None and (tuple(grad.shape) != (N, C) or grad.dtype != z.dtype or not grad.is_contiguous()):
        raise ValueError("grad must be a contiguous [N, C] tensor of the logits' dtype")
    out = dict(H=torch.empty(N, device=z.device), loss=torch.empty(N, device=z.device),
               mean=torch.empty((), device=z.device), kappa=torch.empty(N, dtype=torch.int32, device=z.device),
               grad=torch.empty_like(z) if grad is None else grad)
    rc = lib().fwl_forward_backward_typed(DTYPES[z.dtype], _ptr(z), _ptr(y), N, C, scale, reduce_div, _ptr(out["H"]),
                                          _ptr(out["loss"]), _ptr(out["mean"]), _ptr(out["kappa"]), _ptr(out["grad"]),
                                          _ptr(buf), buf.numel(), _stream())
    _check(rc, "fwl_forward_backward_typed")
    return out


def set_params(path, cand_cap=512):
    _check(lib().fwl_set_params(path, cand_cap), "fwl_set_params")


def forward_backward_ex(z, y, scale=None, reduce_div=None, ws=None, path=None, cand_cap=0, losses64=False,
                        stream=None):
    """fwl_forward_backward_ex: float32/bfloat16/float16 logits whose rows may lie any distance apart
    (z.stride(1) == 1; ld = z.stride(0)), per-call options (path None: the process defaults), and the
    fp64 per-row losses when `losses64`.  Returns dict(H, loss, loss64, mean, kappa, grad)."""
    N, C = z.shape
    if N > 1 and z.stride(1) != 1:
        raise ValueError("the elements of a row must be adjacent (z.stride(1) == 1)")
    ld = z.stride(0) if N > 1 else C
    scale = (1.0 / N if N else 1.0) if scale is None else scale
    reduce_div = float(N) if reduce_div is None else reduce_div
    opt = None if path is None else Options(path, cand_cap)
    ws = ws or Workspace(z.device)
    buf = ws.get(N, C, opt)
    dev = z.device
    out = dict(H=torch.empty(N, device=dev), loss=torch.empty(N, device=dev),
               loss64=torch.empty(N, dtype=torch.float64, device=dev) if losses64 else None,
               mean=torch.empty((), device=dev), kappa=torch.empty(N, dtype=torch.int32, device=dev),
               grad=torch.empty((N, C), dtype=z.dtype, device=dev))
    s = ctypes.c_void_p((stream or torch.cuda.current_stream()).cuda_stream)
    rc = lib().fwl_forward_backward_ex(DTYPES[z.dtype], _ptr(z), ld, _ptr(y), N, C, scale, reduce_div, _ptr(out["H"]),
                                       _ptr(out["loss"]), _ptr(out["loss64"]), _ptr(out["mean"]), _ptr(out["kappa"]),
                                       _ptr(out["grad"]), _ptr(buf), buf.numel(),
                                       None if opt is None else ctypes.byref(opt), s)
    _check(rc, "fwl_forward_backward_ex")
    return out
