"""Host-side checks that need no GPU: the C ABI library and its header, argument validation
(every entry point validates before it touches a device), the torch extension's argument errors,
the synthetic-data generators and the package's separation from the oracle.
"""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

import fwloss_capi as capi
import fwloss_data as data

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "fast-familywise-loss_amd")

# fake device addresses: validation rejects the call before any of them is dereferenced
A16 = 0x10000          # 16-byte aligned
A4 = 0x10004           # 4-byte aligned only
A2 = 0x10002           # misaligned for everything


def P(x):
    return ctypes.c_void_p(x)


def test_library_exports_every_declared_function():
    L = capi.lib()
    declared = capi.declared_functions()
    assert len(declared) == 26
    for name in declared:
        assert hasattr(L, name), name
    # the ctypes signature table covers exactly the header
    assert sorted(capi.SIGNATURES) == declared
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r" T (fwl_\w+)$", out.stdout, re.M))
    assert exported == set(declared)


def test_header_is_plain_c():
    # the boundary must be usable from C (cgo/JNI/ctypes): compile the header alone as C99
    src = '#include "fwloss.h"\nint main(void) { int p, c; return fwl_get_params(&p, &c); }\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                        "-x", "c", "-"], input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_status_strings():
    texts = [capi.status_string(i) for i in range(6)]
    assert texts[0] == "ok"
    assert len(set(texts)) == 6
    assert capi.status_string(99) == "unknown fwloss status"


def ws_round(b):
    return -(-b // 256) * 256


def ws_expect(N, extra=0):
    """The workspace layout: fp64 partials for the two largest grids of a call (>= 4096 blocks
    each, one per 256 rows beyond), the overflow records (two floats per row), then the long rows'
    scratch."""
    slots = 2 * max(-(-N // 256), 4096)
    return ws_round(8 * slots) + ws_round(8 * N) + extra


def test_workspace_bytes():
    L = capi.lib()
    assert L.fwl_workspace_bytes(0, 1) == ws_expect(0)
    assert L.fwl_workspace_bytes(65536, 1000) == ws_expect(65536)
    assert L.fwl_workspace_bytes(1 << 22, 10) == ws_expect(1 << 22)
    assert L.fwl_workspace_bytes(1 << 22, 10) >= L.fwl_workspace_bytes((1 << 22) - 1, 10)
    # per-call options: the same sizes as the process-wide switches; out of range gives 0
    assert L.fwl_workspace_bytes_ex(65536, 1000, None) == ws_expect(65536)
    opt = capi.Options(2, 512)
    assert L.fwl_workspace_bytes_ex(16, 1000, ctypes.byref(opt)) == ws_expect(16, 16 * (512 * 4 + 8))
    for bad in (capi.Options(9, 512), capi.Options(-1, 0), capi.Options(2, 63), capi.Options(2, 513)):
        assert L.fwl_workspace_bytes_ex(16, 1000, ctypes.byref(bad)) == 0


def test_forward_backward_argument_errors():
    L = capi.lib()
    ws_need = L.fwl_workspace_bytes(8, 16)

    def call(z=A16, y=A16, N=8, C=16, H=A16, loss=A16, mean=A16, kappa=A16, grad=A16, ws=A16, wsb=ws_need):
        return L.fwl_forward_backward(P(z), P(y), N, C, 1.0, 1.0, P(H), P(loss), P(mean), P(kappa), P(grad),
                                      P(ws), wsb, None)
    assert call(z=None) == 1
    assert call(y=None) == 1
    assert call(grad=None) == 1
    assert call(N=-1) == 1
    assert call(C=0) == 1
    assert call(C=2 ** 31) == 1
    assert call(C=2 ** 29 + 1) == 1
    assert call(z=A2) == 3
    assert call(y=A4) == 3
    assert call(grad=A2) == 3
    assert call(ws=None) == 2
    assert call(wsb=ws_round(8 * 2 * 4096) - 1) == 2     # the mean needs its partials
    assert call(ws=A4 + 2) == 2


def test_ex_entry_point_argument_errors():
    L = capi.lib()
    ws_need = L.fwl_workspace_bytes(8, 16)

    def call(dtype=0, z=A16, ld=16, N=8, C=16, l64=A16, grad=A16, opt=None):
        return L.fwl_forward_backward_ex(dtype, P(z), ld, P(A16), N, C, 1.0, 1.0, P(A16), P(A16), P(l64), P(A16),
                                         P(A16), P(grad), P(A16), ws_need, opt, None)
    assert call(ld=15) == 1                     # rows overlap
    assert call(ld=2 ** 29 + 1) == 1
    assert call(dtype=3) == 1
    assert call(grad=None) == 1
    assert call(dtype=1, z=A16 + 1) == 3
    for bad in (capi.Options(9, 0), capi.Options(-1, 0), capi.Options(3, 32), capi.Options(3, 1024)):
        assert call(opt=ctypes.byref(bad)) == 1


def test_other_entry_point_argument_errors():
    L = capi.lib()
    ws_need = L.fwl_workspace_bytes(8, 16)
    assert L.fwl_forward_small(P(A16), P(A16), 8, 16, P(A16), P(A16), P(A16), P(A16), None, P(A16), ws_need,
                               None) == 1
    assert L.fwl_forward_small(P(A16), P(A16), 8, 16, P(A16), P(A16), P(A16), P(A16), P(A16), P(A16), 8,
                               None) == 2
    assert L.fwl_forward_large(P(A16), P(A16), 8, 16, P(A16), P(A16), P(A16), P(A16), P(A16), None, P(A16),
                               P(A16), ws_need, None) == 1
    assert L.fwl_forward_large(P(A16), P(A16), 8, 16, P(A16), P(A16), P(A16), P(A16), P(A2), P(A16), P(A16),
                               P(A16), ws_need, None) == 3
    assert L.fwl_backward_small(P(A16), P(A16), None, 8, 16, P(A16), None) == 1
    assert L.fwl_backward_small(P(A4), P(A16), P(A16), 8, 16, P(A16), None) == 3
    assert L.fwl_backward_large(P(A16), P(A16), P(A16), P(A16), P(A16), P(A16), None, 8, 16, P(A16), None) == 1
    assert L.fwl_backward_large(P(A16), P(A16), P(A16), P(A16), P(A16), P(A16), P(A16), 8, 16, P(A2), None) == 3
    assert L.fwl_scale_grad(P(A16), P(A16), -1, 8, 16, None) == 1
    assert L.fwl_scale_grad(P(A16), None, 0, 8, 16, None) == 1
    assert L.fwl_scale_grad(P(A2), P(A16), 0, 8, 16, None) == 3
    # empty batches return before any launch for the backward entry points
    assert L.fwl_backward_small(None, None, None, 0, 16, None, None) == 0
    assert L.fwl_scale_grad(None, None, 0, 0, 16, None) == 0


def test_typed_entry_point_argument_errors():
    L = capi.lib()
    ws_need = L.fwl_workspace_bytes(8, 16)

    def call(dtype=1, z=A16, grad=A16, N=8, C=16):
        return L.fwl_forward_backward_typed(dtype, P(z), P(A16), N, C, 1.0, 1.0, P(A16), P(A16), P(A16), P(A16),
                                            P(grad), P(A16), ws_need, None)
    assert call(dtype=3) == 1
    assert call(dtype=-1) == 1
    assert call(grad=None) == 1
    assert call(z=A16 + 1) == 3               # 16-bit logits need 2-byte alignment
    assert call(grad=A16 + 1) == 3
    assert call(dtype=0, z=A16 + 2) == 3       # fp32 logits need 4
    assert L.fwl_scale_grad_typed(5, P(A16), P(A16), 0, 8, 16, None) == 1
    assert L.fwl_scale_grad_typed(2, P(A16 + 1), P(A16), 0, 8, 16, None) == 3
    assert L.fwl_scale_grad_typed(1, None, None, 0, 0, 16, None) == 0


def test_linear_entry_point_argument_errors():
    L = capi.lib()
    assert L.fwl_linear_state_bytes(10) == 10 * (32 + 8 * L.fwl_linear_support_cap())
    assert L.fwl_linear_state_bytes(0) == 0
    assert L.fwl_linear_begin(None, 8, None) == 1
    assert L.fwl_linear_begin(P(A16 + 8), 8, None) == 3          # the state needs 16-byte alignment
    assert L.fwl_linear_begin(None, 0, None) == 0

    def chunk(dtype=1, z=A16, N=8, Vc=16, ld=16, v0=0, V=64, y=A16, st=A16):
        return L.fwl_linear_chunk(dtype, P(z), N, Vc, ld, v0, V, P(y), P(st), None)
    assert chunk(dtype=3) == 1
    assert chunk(ld=15) == 1                   # rows shorter than the chunk
    assert chunk(v0=60) == 1                   # columns past V
    assert chunk(v0=-1) == 1
    assert chunk(z=None) == 1
    assert chunk(y=A16 + 4) == 3
    assert chunk(z=A16 + 1) == 3               # 16-bit logits need 2-byte alignment
    assert chunk(N=0) == 0
    assert L.fwl_linear_finish(P(A16), P(A16), 8, 0, P(A16), P(A16), P(A16), P(A16), P(A16), None) == 1
    assert L.fwl_linear_finish(P(A16), P(A16), 8, 64, P(A16), None, P(A16), P(A16), P(A16), None) == 1
    assert L.fwl_linear_finish(P(A16), P(A16), 8, 64, P(A16), P(A16), P(A16), P(A16 + 2), P(A16), None) == 3
    assert L.fwl_linear_dhidden(1, P(A16), 64, 0, P(A16), P(A16), P(A16), P(A16), 0, 8, P(A16), None) == 1
    assert L.fwl_linear_dhidden(1, P(A16), 64, 32, P(A16), P(A16), P(A16), P(A16), -1, 8, P(A16), None) == 1
    assert L.fwl_linear_dhidden(4, P(A16), 64, 32, P(A16), P(A16), P(A16), P(A16), 0, 8, P(A16), None) == 1
    assert L.fwl_linear_dhidden(1, P(A16 + 1), 64, 32, P(A16), P(A16), P(A16), P(A16), 0, 8, P(A16), None) == 3
    assert L.fwl_linear_coo(P(A16), 8, 64, P(A16), P(A16), None, P(A16), 0, P(A16), P(A16), None) == 1
    assert L.fwl_linear_coo(P(A16), 8, 64, P(A16), P(A16), P(A16), P(A16), 0, P(A16 + 4), P(A16), None) == 3
    assert L.fwl_linear_dweight(1, P(A16), 8, 64, 32, None, P(A16), 5, P(A16), None) == 1
    assert L.fwl_linear_dweight(1, P(A16), 8, 0, 32, P(A16), P(A16), 5, P(A16), None) == 1
    assert L.fwl_linear_dweight(1, P(A16), 8, 64, 32, P(A16), P(A16), 0, P(A16), None) == 0


def test_linear_loss_rejects_cpu_and_bad_arguments():
    import fwloss
    h, w, y = torch.zeros(4, 8), torch.zeros(10, 8), torch.zeros(4, dtype=torch.long)
    with pytest.raises(RuntimeError, match="CUDA"):
        fwloss.familywise_linear_loss(h, w, y)
    with pytest.raises(KeyError):
        fwloss.familywise_linear_loss(h, w, y, reduction="max")


def test_set_params_validation_and_round_trip():
    L = capi.lib()
    p, c = ctypes.c_int(-1), ctypes.c_int(-1)
    assert L.fwl_get_params(ctypes.byref(p), ctypes.byref(c)) == 0
    saved = (p.value, c.value)
    try:
        assert L.fwl_set_params(9, 512) == 1
        assert L.fwl_set_params(8, 512) == 0
        assert L.fwl_set_params(7, 512) == 0
        assert L.fwl_set_params(-1, 512) == 1
        assert L.fwl_set_params(2, 63) == 1
        assert L.fwl_set_params(2, 513) == 1
        assert L.fwl_set_params(2, 64) == 0
        L.fwl_get_params(ctypes.byref(p), ctypes.byref(c))
        assert (p.value, c.value) == (2, 64)
    finally:
        L.fwl_set_params(*saved)


def test_workspace_sizes():
    """The split-row scratch is counted exactly where the split kernels may run: few rows (<= 128)
    of at least 96 KiB (24576 fp32 elements; the size covers every element type), or rows of any
    length when path 7 is forced; the two-pass scratch where the fused op may run in two passes
    (>= 384 rows of >= 32000 elements, rows of >= 8192 elements in batches of >= 32M elements, or
    path 2/3 forced).  The two share one region (the larger is counted)."""
    L = capi.lib()
    p, c = ctypes.c_int(-1), ctypes.c_int(-1)
    L.fwl_get_params(ctypes.byref(p), ctypes.byref(c))
    saved = (p.value, c.value)
    W = L.fwl_workspace_bytes
    try:
        L.fwl_set_params(0, 512)
        assert W(16, 1000) == ws_expect(16)           # short rows: no scratch
        assert W(65536, 8191) == ws_expect(65536)
        assert W(0, 131072) == ws_expect(0)
        # >= 384 rows of >= 32000 elements, or batches of >= 32M elements in rows of >= 8192 (the
        # fp32 rules, which cover the 16-bit ones) run the fused op in two passes: per row 512
        # support indices, the read pass's count and H
        row = 512 * 4 + 4 + 4
        assert W(2048, 131072) == ws_expect(2048, 2048 * row)
        assert W(384, 32000) == ws_expect(384, 384 * row)
        assert W(383, 32000) == ws_expect(383)
        assert W(4096, 8192) == ws_expect(4096, 4096 * row)      # 32M elements
        assert W(4095, 8192) == ws_expect(4095)
        assert W(6144, 8191) == ws_expect(6144)
        # 16-bit rows without 128-bit units take two passes from 12000 elements at 8 rows per CU
        # (the count follows the device's CUs: 256 on MI355X, and 256 without a device)
        cus = 256
        assert W(8 * cus, 12000) == ws_expect(8 * cus, 8 * cus * row)
        assert W(8 * cus - 1, 12000) == ws_expect(8 * cus - 1)
        assert W(8 * cus, 11999) == ws_expect(8 * cus)
        assert W(65536, 8192) == ws_expect(65536, 65536 * row)
        assert W(1024, 31999) == ws_expect(1024)
        assert W(129, 24576) == ws_expect(129)
        assert W(128, 24575) == ws_expect(128)
        # (row, chunk) items: about 1024 in all, chunks of at least 4096 elements, <= 256 per row;
        # per item tau_c (8), the support size (4), the chunk maximum (4), 64 values and indices
        item = 8 + 4 + 4 + 64 * 8
        assert W(16, 131072) == ws_expect(16, 16 * 32 * item)
        assert W(3, 131072) == ws_expect(3, 3 * 32 * item)
        assert W(1, 2 ** 29) == ws_expect(1, 1 * 256 * item)
        assert W(128, 24576) == ws_expect(128, 128 * 6 * item)
        assert W(100, 40000) == ws_expect(100, 100 * 10 * item)
        L.fwl_set_params(2, 512)                                  # forced block path: two passes
        assert W(16, 1000) == ws_expect(16, 16 * row)
        L.fwl_set_params(7, 512)
        assert W(16, 1000) == ws_expect(16, 16 * 1 * item)
        assert W(4, 30000) == ws_expect(4, 4 * 8 * item)
        assert W(129, 30000) == ws_expect(129)                    # more rows than path 7 takes
    finally:
        L.fwl_set_params(*saved)


def test_extension_rejects_cpu_and_bad_inputs():
    import fwloss
    z = torch.zeros(4, 6)
    y = torch.zeros(4, dtype=torch.long)
    for op in (fwloss.fw_forward_small, fwloss.fw_forward, fwloss.fw_forward_backward):
        with pytest.raises(RuntimeError, match="logits must be a CUDA tensor"):
            op(z, y)
    with pytest.raises(RuntimeError, match="CUDA"):
        fwloss.familywise_loss(z, y)
    with pytest.raises(ValueError, match="Invalid reduction mode"):
        fwloss.familywise_loss(z, y, reduction="max")
    with pytest.raises(KeyError):   # what the reference's dict lookup raises (src/cpu/fwcpp.py:19)
        fwloss.familywise_loss(z, y, reduction="max")
    with pytest.raises(RuntimeError):
        fwloss.set_params(9, 512)
    assert tuple(fwloss.get_params()) == (0, 512)
    libs = fwloss.native_libraries()
    assert any(p.endswith("libfwloss.so") for p in libs) and any("fw_radix_cuda" in p for p in libs)


@pytest.mark.parametrize("cfg", sorted(data.CONFIGS))
def test_generators(cfg):
    z, y = data.make(cfg, N=16, seed=5)
    C = data.CONFIGS[cfg]["C"]
    assert z.shape == (16, C) and z.dtype == np.float32 and z.flags.c_contiguous
    assert y.shape == (16,) and y.dtype == np.int64 and y.min() >= 0 and y.max() < C
    z2, y2 = data.make(cfg, N=16, seed=5)
    np.testing.assert_array_equal(z, z2)
    np.testing.assert_array_equal(y, y2)
    assert not np.array_equal(z, data.make(cfg, N=16, seed=6)[0])


def test_edge_rows():
    z, y = data.edge_rows()
    assert z.dtype == np.float32 and z.shape[0] == y.shape[0] >= 10
    assert (y >= 0).all() and (y < z.shape[1]).all()
    assert np.isneginf(z).any() and (np.abs(z) >= 2.0 ** 53).any()


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_product_never_touches_the_oracle():
    """Only tests, smoke() and bench.py's CPU baseline may use oracle/; the package never does."""
    for dirpath, _, files in os.walk(PKG):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                with open(os.path.join(dirpath, f)) as fh:
                    text = fh.read()
                assert not re.search(r"^\s*(import|from)\s+oracle\b", text, re.M), f
                assert "fwl_oracle" not in text and "oracle/" not in text, f
