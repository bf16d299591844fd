"""fwl_forward_backward_noalloc: the fused op with the library's static device scratch instead of a
workspace (for callers that cannot allocate).  Its outputs equal those of fwl_forward_backward_ex
with a workspace, bit for bit, on two calls in a row (the second one smaller, so that it runs over
what the first left in the scratch), across the kernel families; sizes beyond the scratch are
refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

import fwloss_capi
import fwloss_data as data

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p


def noalloc(z, y, scale=None, rdiv=None, path=None):
    N, C = z.shape
    dev = z.device
    out = dict(H=torch.empty(N, device=dev), loss=torch.empty(N, device=dev),
               loss64=torch.empty(N, dtype=torch.float64, device=dev), mean=torch.empty((), device=dev),
               kappa=torch.empty(N, dtype=torch.int32, device=dev), grad=torch.empty((N, C), dtype=z.dtype, device=dev))
    opt = None if path is None else fwloss_capi.Options(path, 0)
    rc = fwloss_capi.lib().fwl_forward_backward_noalloc(
        fwloss_capi.DTYPES[z.dtype], P(z.data_ptr()), z.stride(0) if N > 1 else C, P(y.data_ptr()), N, C,
        (1.0 / N if N else 1.0) if scale is None else scale, float(N) if rdiv is None else rdiv,
        P(out["H"].data_ptr()), P(out["loss"].data_ptr()), P(out["loss64"].data_ptr()), P(out["mean"].data_ptr()),
        P(out["kappa"].data_ptr()), P(out["grad"].data_ptr()), None if opt is None else ctypes.byref(opt),
        P(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, fwloss_capi.status_string(rc)
    return out


def same(a, b):
    for k in ("H", "loss", "loss64", "mean", "kappa", "grad"):
        x, y = a[k].cpu(), b[k].cpu()
        assert torch.equal(x.view(-1).view(torch.int32 if x.element_size() == 4 else
                                           (torch.int64 if x.element_size() == 8 else torch.int16)),
                           y.view(-1).view(torch.int32 if y.element_size() == 4 else
                                           (torch.int64 if y.element_size() == 8 else torch.int16))), k


@pytest.mark.parametrize("shapes", [
    [("cfg2", 4096, 1000, 1.0), ("cfg2", 1000, 1000, 1.0)],        # register rows
    [("gauss", 700, 3000, 0.001), ("gauss", 300, 3000, 1.0)],      # streaming, overflow kernel
    [("gauss", 400, 32000, 1.0), ("gauss", 390, 32000, 0.01)],     # two passes
    [("gauss", 16, 131072, 1.0), ("gauss", 3, 131072, 0.001)],     # split rows
    [("cfg3", 16384, 100, 1.0), ("cfg3", 100, 100, 1.0)],          # segmented short rows
])
def test_noalloc_matches_workspace_entry_point(dev, shapes):
    for (kind, N, C, sigma) in shapes:
        if kind.startswith("cfg"):
            z, y = data.make(kind, N=N, seed=N)
            z = z[:, :C]
        else:
            z, y = data.make_dist(kind, N, C, sigma, seed=N)
        zt = torch.from_numpy(np.ascontiguousarray(z)).to(dev)
        yt = torch.from_numpy(y).to(dev)
        print(f"noalloc {kind} N={N} C={C} sigma={sigma}", flush=True)
        a = noalloc(zt, yt)
        b = fwloss_capi.forward_backward_ex(zt, yt, losses64=True)
        torch.cuda.synchronize()
        same(a, b)


def test_noalloc_16bit_and_strided(dev):
    rng = np.random.default_rng(3)
    for dt in (torch.bfloat16, torch.float16):
        wide = torch.from_numpy(rng.standard_normal((300, 1003)).astype(np.float32)).to(dev).to(dt)
        zt = wide[:, 3:]
        yt = torch.from_numpy(rng.integers(0, 1000, 300)).to(dev)
        a = noalloc(zt, yt)
        b = fwloss_capi.forward_backward_ex(zt, yt, losses64=True)
        torch.cuda.synchronize()
        same(a, b)


def test_noalloc_refuses_sizes_beyond_the_scratch(dev):
    L = fwloss_capi.lib()
    cap = L.fwl_noalloc_scratch_bytes()
    assert cap == 64 << 20
    N = 12 << 20                                 # overflow records alone exceed 64 MiB
    assert L.fwl_workspace_bytes(N, 16) > cap
    rc = L.fwl_forward_backward_noalloc(0, P(0x10000), 16, P(0x10000), N, 16, 1.0, 1.0, None, None, None,
                                        P(0x10000), None, P(0x10000), None, None)
    assert rc == 2                               # FWL_ERR_WORKSPACE, before any launch
    assert L.fwl_workspace_bytes(1 << 20, 16) <= cap
