"""Familywise (FW) loss on MI355X: the Python API over the ``fw_radix_cuda`` extension.

Mirrors the reference's CPU module ``src/cpu/fwcpp.py:18-26``::

    from fwloss import familywise_loss
    loss = familywise_loss(logits, target, reduction="mean")   # logits: float32 [N, C] on the GPU
    loss.backward()

The forward runs the fused HIP kernel, which computes the loss and the gradient in one pass over
the logits (as the reference's C++ autograd Function does eagerly, src/cpu/fw_cpu.cpp:721-733);
the backward multiplies the stored gradient by ``grad_output`` on the device, skipping rows whose
factor is 1 (fw_cpu.cpp:734-740).  There is no CPU fallback: without the HIP extension the import
fails, and CPU tensors are rejected.

The reference GPU ops are re-exported unchanged: ``fw_forward``, ``fw_backward``,
``fw_forward_small``, ``fw_backward_small`` (src/cuda/binding.cpp:8-13).
"""
import os
import sys

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

try:
    import fw_radix_cuda as _ext  # noqa: E402  (torch must be imported first: one HIP runtime)
except ImportError as e:  # pragma: no cover - exercised only on a broken install
    raise ImportError("fw_radix_cuda is not built; run `python fast-familywise-loss_amd/fwloss_build.py` "
                      "(there is no CPU fallback)") from e

fw_forward = _ext.fw_forward
fw_backward = _ext.fw_backward
fw_forward_small = _ext.fw_forward_small
fw_backward_small = _ext.fw_backward_small
fw_forward_backward = _ext.fw_forward_backward
set_params = _ext.set_params
get_params = _ext.get_params

_REDUCTIONS = ("mean", "sum", "none")


class ReductionError(KeyError, ValueError):
    """Unknown reduction name.  The reference looks the name up in a dict (src/cpu/fwcpp.py:19) and
    so raises KeyError; this is also a ValueError, the usual type for a bad argument value."""

    def __str__(self):
        return str(self.args[0]) if self.args else ""


class FWFunction(torch.autograd.Function):
    """Eager-gradient autograd Function (the GPU counterpart of fw_cpu.cpp:721-741).  The backward
    scales the stored gradient in place and hands it over, so it runs once per forward, like the
    reference's, which erases the stored gradient (fw_cpu.cpp:734-740); a second backward through
    the same graph raises instead of returning a gradient scaled twice."""

    @staticmethod
    def forward(ctx, logits, target, reduction):
        N = logits.shape[0]
        if reduction == "mean":
            scale, rdiv = (1.0 / N if N else 1.0), float(N)
        else:
            scale, rdiv = 1.0, 1.0
        _, losses, reduced, _, grad = _ext.fw_forward_backward(logits.detach(), target, scale, rdiv)
        ctx.save_for_backward(grad)
        ctx.consumed = False
        # the loss has the logits' dtype, as in the reference (fw_cpu.cpp:732); computed in fp32/fp64
        out = losses if reduction == "none" else reduced
        return out if out.dtype == logits.dtype else out.to(logits.dtype)

    @staticmethod
    def backward(ctx, grad_output):
        if ctx.consumed:
            raise RuntimeError("familywise_loss: the backward of this loss already ran (its stored gradient was "
                               "scaled in place and handed over); compute the loss again for another backward")
        (grad,) = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None
        ctx.consumed = True
        _ext.fw_scale_grad(grad, grad_output.detach())
        return grad, None, None


def familywise_loss(logits, target, reduction="mean"):
    """FW loss of logits [N, C] (GPU; float32, float64, bfloat16 or float16) and int64 targets
    [N]; reduction 'mean' | 'sum' | 'none'.  16-bit logits are widened to fp32 exactly; float64
    logits are decided in fp64 (the reference CPU path's two dtypes, src/cpu/fw_cpu.cpp:697-703).
    The loss and the gradient are returned in the logits' dtype (16-bit gradients rounded to
    nearest-even).

    Same call shape as the reference's ``fwcpp.familywise_loss`` (src/cpu/fwcpp.py:18-19), which
    accepts 'sum' and 'mean'; 'none' returns the per-row losses (reference_impl.py:30-33).
    """
    if reduction not in _REDUCTIONS:
        raise ReductionError(f"Invalid reduction mode: {reduction!r} (expected 'mean', 'sum' or 'none')")
    if not logits.is_cuda:
        raise RuntimeError("familywise_loss: logits must be a CUDA (ROCm) tensor; this package has no CPU path")
    return FWFunction.apply(logits, target, reduction)


def fw_loss_grad(Z, y, scale=1.0, flat_kmax=None, serial_below=None, use_chunked=None):
    """(per-row loss [N] float64, scale * gradient [N, C] in Z's dtype, kappa [N] int64), the outputs
    and dtypes of fwcpp.fw_loss_grad (src/cpu/fwcpp.py:21-23).  flat_kmax, serial_below and
    use_chunked tune the reference's CPU branches (fw_cpu.cpp:750-757); they are accepted and have
    no effect here.  The losses are the kernel's fp64 values (1 - z_y) + tau, not rounded to fp32."""
    if not Z.is_cuda:
        raise RuntimeError("fw_loss_grad: Z must be a CUDA (ROCm) tensor")
    out = _ext.fw_forward_backward(Z, y, float(scale), 1.0, losses64=True)
    return out[5], out[4], out[3].long()


def linear_forward(hidden, weight, target, chunk=8192):
    """The loss side of ``familywise_linear_loss``: logits = hidden @ weight.T one vocabulary chunk
    of ``chunk`` columns at a time (each chunk's logits exist only while it is merged), then the
    threshold of every row from its carried list.  Returns a dict with H, losses, kappa (int32),
    support (int32 [N, cap], the first kappa entries valid), overflow (rows solved on their
    materialised logits instead) and dense = (rows, grad of those rows with scale 1) or None.
    H, losses and kappa are those ``fw_forward_backward`` gives on the concatenated chunk logits."""
    if not (hidden.is_cuda and weight.is_cuda):
        raise RuntimeError("familywise_linear_loss: hidden and weight must be CUDA (ROCm) tensors")
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError("hidden must be [N, d] and weight [V, d]")
    if chunk < 1:
        raise ValueError("chunk must be >= 1")
    N, V = hidden.shape[0], weight.shape[0]
    h = hidden.detach().contiguous()
    w = weight.detach().contiguous()
    y = target.contiguous()
    state = _ext.fw_linear_state(h, N)
    for v0 in range(0, V, chunk):
        _ext.fw_linear_chunk(state, torch.nn.functional.linear(h, w[v0:v0 + chunk]), y, v0, V)
    H, losses, kappa, support, overflow = _ext.fw_linear_finish(state, y, V)
    rows = overflow.nonzero().flatten()
    dense = None
    kappa_sparse = kappa
    if rows.numel():
        # rows whose lists outgrew the state: their logits in full, through the fused op
        Hr, lr, _, kr, gr = _ext.fw_forward_backward(torch.nn.functional.linear(h[rows], w), y[rows], 1.0, 1.0)
        H[rows] = Hr
        losses[rows] = lr
        kappa_sparse = kappa.clone()   # 0: the sparse gradient kernels skip these rows
        kappa[rows] = kr
        dense = (rows, gr)
    return {"H": H, "losses": losses, "kappa": kappa, "kappa_sparse": kappa_sparse, "support": support,
            "overflow": overflow, "dense": dense}


class FWLinearFunction(torch.autograd.Function):
    """FW loss of hidden @ weight.T without materialising the logits.  The gradient with respect to
    the logits has kappa + 1 non-zeros per row, so the backward gathers and scatters weight and
    hidden rows instead of running the two GEMMs of an unfused backward."""

    @staticmethod
    def forward(ctx, hidden, weight, target, reduction, chunk):
        res = linear_forward(hidden, weight, target, chunk)
        losses = res["losses"]
        N = hidden.shape[0]
        if reduction == "none":
            out = losses
        else:
            total = losses.double().sum()
            out = (total / N if reduction == "mean" else total).float()   # an empty mean is NaN
        ctx.save_for_backward(hidden.detach(), weight.detach(), target, res["kappa_sparse"], res["support"])
        ctx.dense = res["dense"]
        ctx.reduction = reduction
        return out.to(hidden.dtype)

    @staticmethod
    def backward(ctx, grad_output):
        h, w, y, kappa, support = ctx.saved_tensors
        want_dh, want_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (want_dh or want_dw):
            return None, None, None, None, None
        N = h.shape[0]
        go = grad_output.detach().float()
        if ctx.reduction == "mean":
            rs = (go / N if N else go).reshape(1)
        else:
            rs = go.reshape(-1)
        dh, dw = _ext.fw_linear_grads(h, w, y, kappa, support, rs, want_dh, want_dw)
        if ctx.dense is not None:
            # rows solved on their materialised logits: dense logit gradients, in the weight's dtype
            rows, gr = ctx.dense
            g = (gr.float() * (rs if rs.numel() == 1 else rs[rows]).reshape(-1, 1)).to(w.dtype)
            if want_dh:
                dh.index_add_(0, rows, g @ w)
            if want_dw:
                dw.addmm_(g.t().contiguous(), h[rows])
        return (dh if want_dh else None), (dw if want_dw else None), None, None, None


def familywise_linear_loss(hidden, weight, target, reduction="mean", chunk=8192):
    """FW loss of the logits hidden @ weight.T (an LM head: hidden [N, d], weight [V, d], one dtype:
    float32, bfloat16 or float16) and int64 targets [N], computed one vocabulary chunk of
    ``chunk`` columns at a time.  The loss equals ``familywise_loss(hidden @ weight.T, target,
    reduction)`` on the same chunk logits; the gradients of hidden and weight come from the
    loss's sparse logit gradient (kappa + 1 non-zeros per row) without an [N, V] tensor."""
    if reduction not in _REDUCTIONS:
        raise ReductionError(f"Invalid reduction mode: {reduction!r} (expected 'mean', 'sum' or 'none')")
    return FWLinearFunction.apply(hidden, weight, target, reduction, chunk)


def native_libraries():
    """Paths of the native libraries this module runs on (for load checks)."""
    return [os.path.join(_HERE, "libfwloss.so"), _ext.__file__]
