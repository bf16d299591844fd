"""bfloat16 / float16 logits through the fused op (fwl_forward_backward_typed) and the autograd API.

The expected values are the fp32 oracle's on the widened inputs (16-bit values are exact in fp32),
with the gradient rounded to the logits' dtype by torch's own CPU conversion (round to nearest
even, subnormals kept) -- an implementation independent of the kernel's.  Bar: kappa, H, losses
bit-identical; the gradient bit-identical in the 16-bit dtype; the mean within 1e-6 relative.
"""
import numpy as np
import pytest
import torch

import fwloss_capi
import oracle

pytestmark = pytest.mark.gpu

DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16}


def case(C, N, seed, dtype):
    """Seeded rows in the 16-bit dtype: N(0,1) scaled per row, every 7th row flat, some dyadic ties."""
    rng = np.random.default_rng(seed)
    z = rng.standard_normal((N, C)) * rng.choice([0.05, 1.0, 4.0], size=(N, 1))
    z[::7] *= 0.01
    z[3::11] = np.round(z[3::11] * 2) / 2
    z16 = torch.from_numpy(z.astype(np.float32)).to(dtype)
    y = rng.integers(0, C, N)
    return z16, y


def expected(z16, y, scale):
    z32 = z16.float().numpy()
    ref = oracle.definition(z32, y, scale=scale)
    g16 = torch.from_numpy(ref["grad"]).to(z16.dtype)
    return ref, g16


def check(ext, dev, z16, y, scale=-1.0, rdiv=-1.0):
    N = z16.shape[0]
    zt, yt = z16.to(dev), torch.from_numpy(y).to(dev)
    H, loss, mean, kappa, grad = ext.fw_forward_backward(zt, yt, scale, rdiv)
    torch.cuda.synchronize()
    assert grad.dtype == z16.dtype and H.dtype == torch.float32 and loss.dtype == torch.float32
    sc = (1.0 / N if N else 1.0) if scale < 0 else scale
    ref, g16 = expected(z16, y, sc)
    np.testing.assert_array_equal(kappa.cpu().numpy(), ref["kappa"])
    np.testing.assert_array_equal(H.cpu().numpy().view(np.uint32), ref["H"].view(np.uint32))
    np.testing.assert_array_equal(loss.cpu().numpy().view(np.uint32), ref["loss"].view(np.uint32))
    got = grad.cpu()
    assert torch.equal(got.view(torch.int16), g16.view(torch.int16)), "grad not bit-identical in the 16-bit dtype"
    if rdiv < 0 and N:
        assert abs(float(mean.cpu()) - ref["mean"]) <= 1e-6 * max(1.0, abs(ref["mean"]))


@pytest.mark.parametrize("name", sorted(DTYPES))
@pytest.mark.parametrize("C", [1, 10, 64, 100, 128, 256, 512, 1000, 1024, 2048, 2999, 3000, 8200, 20000])
def test_dtype_shapes(ext, dev, name, C):
    N = 96 if C >= 8192 else 300
    z16, y = case(C, N, C + 5, DTYPES[name])
    print(f"{name} C={C} N={N}", flush=True)
    check(ext, dev, z16, y)


@pytest.mark.parametrize("name", sorted(DTYPES))
@pytest.mark.parametrize("N,C", [(300, 130), (300, 1002), (300, 2046), (300, 2050), (200, 3002), (96, 8194),
                                 (1030, 12002), (96, 30002), (16, 50002), (600, 65538)])
def test_dtype_even_rows(ext, dev, name, N, C):
    """16-bit rows of even length that are not whole 128-bit units run 128-bit accesses with the
    per-dword range check (register rows, streamed rows, one block per row, split rows, two
    passes)."""
    z16, y = case(C, N, N * 7 + C, DTYPES[name])
    print(f"{name} even N={N} C={C}", flush=True)
    check(ext, dev, z16, y)


@pytest.mark.parametrize("name", sorted(DTYPES))
@pytest.mark.parametrize("path", [1, 2, 4, 7])
def test_dtype_even_rows_forced(ext, dev, reset_params16, name, path):
    z16, y = case(3002, 64, 3002 + path, DTYPES[name])
    ext.set_params(path, 512)
    check(ext, dev, z16, y)


@pytest.mark.parametrize("name", sorted(DTYPES))
@pytest.mark.parametrize("N,C", [(1024, 8193), (1100, 12000), (1030, 28672), (1023, 20000), (1500, 28673)])
def test_dtype_long_rows_streamed(ext, dev, name, N, C):
    """16-bit rows of 8193-28672 elements stream on one wavefront each from 1024 rows on (one block
    per row below that and beyond 28672); both sides of both boundaries."""
    z16, y = case(C, N, N + C, DTYPES[name])
    print(f"{name} N={N} C={C}", flush=True)
    check(ext, dev, z16, y)


@pytest.mark.parametrize("name", sorted(DTYPES))
@pytest.mark.parametrize("path,cap", [(1, 512), (2, 512), (2, 64), (3, 512), (4, 512), (4, 64), (5, 512), (6, 512)])
def test_dtype_forced_paths(ext, dev, reset_params16, name, path, cap):
    z16, y = case(1000, 200, 77, DTYPES[name])
    print(f"{name} path={path} cap={cap}", flush=True)
    ext.set_params(path, cap)
    check(ext, dev, z16, y)


@pytest.mark.parametrize("name", sorted(DTYPES))
@pytest.mark.parametrize("N,C,path", [(40, 20000, 7), (16, 50000, 0), (3, 131072, 0), (16, 40000, 0)])
def test_dtype_split_rows(ext, dev, reset_params16, name, N, C, path):
    # few long rows: forced split, and the automatic rule (rows of >= 96 KiB: 49152 16-bit elements;
    # 40000 elements run one block per row)
    z16, y = case(C, N, C + N, DTYPES[name])
    print(f"{name} split rows N={N} C={C} path={path}", flush=True)
    ext.set_params(path, 512)
    check(ext, dev, z16, y)


@pytest.mark.parametrize("name", sorted(DTYPES))
@pytest.mark.parametrize("N,C,last", [(3, 999, "free"), (5, 7, "label"), (7, 33, "support"), (1, 1, "label")])
def test_dtype_two_pass_odd_sizes(ext, dev, reset_params16, name, N, C, last):
    # forced two passes with a 16-bit gradient of an odd number of elements: the zero fill writes
    # whole dwords, the last element comes from the scatter (as a free entry, the label, or a
    # support entry)
    z16, y = case(C, N, N * 100 + C, DTYPES[name])
    if last == "label":
        y[-1] = C - 1
    elif last == "support":
        z = z16.float()
        z[-1, -1] = z[-1].max() + 2.0     # the row's only support entry
        z16 = z.to(DTYPES[name])
        y[-1] = 0
    else:
        y[-1] = 0
    print(f"{name} two passes odd N={N} C={C} last={last}", flush=True)
    ext.set_params(2, 512)
    check(ext, dev, z16, y)


@pytest.mark.parametrize("name", sorted(DTYPES))
def test_dtype_two_pass(ext, dev, name):
    # >= 512 16-bit rows of >= 65536 elements: the fused op in two passes (read, then write)
    z16, y = case(65536, 512, 21, DTYPES[name])
    print(f"{name} two passes N=512 C=65536", flush=True)
    check(ext, dev, z16, y)


@pytest.mark.parametrize("name", sorted(DTYPES))
@pytest.mark.parametrize("K", [3, 100, 1000, 40000])
def test_dtype_row_families(ext, dev, name, K):
    # every row family, rounded to the 16-bit dtype (which adds many exact ties)
    import fwloss_data as data
    z, y, _ = data.families(K, rows=3, seed=K + 7)
    z16 = torch.from_numpy(z).to(DTYPES[name])
    print(f"{name} families K={K}", flush=True)
    check(ext, dev, z16, y)


@pytest.mark.parametrize("name", sorted(DTYPES))
def test_dtype_subnormal_gradients(ext, dev, name):
    # scale 1e-6: scale/kappa is subnormal in float16 and tests the rounding there
    z16, y = case(512, 64, 3, DTYPES[name])
    print(f"{name} subnormal scale", flush=True)
    check(ext, dev, z16, y, scale=1e-6, rdiv=1.0)


@pytest.mark.parametrize("name", sorted(DTYPES))
def test_dtype_special_values(ext, dev, name):
    dt = DTYPES[name]
    z = np.zeros((6, 16), np.float32)
    z[0] = np.linspace(-2, 2, 16)
    z[1, :] = 1.0                      # constant row
    z[2, 3] = -np.inf                  # -inf entry
    z[3, ::2] = 5.0                    # ties at the top
    z[4] = -0.0
    z[4, 5] = 0.0
    z[5] = np.arange(16) * 0.125       # exact dyadic steps
    z16 = torch.from_numpy(z).to(dt)
    y = np.array([0, 1, 4, 2, 5, 15])
    print(f"{name} special values", flush=True)
    check(ext, dev, z16, y)


@pytest.mark.parametrize("name", sorted(DTYPES))
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_dtype_autograd(ext, dev, name, reduction):
    dt = DTYPES[name]
    z16, y = case(1000, 128, 9, dt)
    zt = z16.to(dev).requires_grad_(True)
    yt = torch.from_numpy(y).to(dev)
    loss = ext.familywise_loss(zt, yt, reduction)
    assert loss.dtype == dt
    N = z16.shape[0]
    scale = 1.0 / N if reduction == "mean" else 1.0
    ref, g16 = expected(z16, y, scale)
    if reduction == "none":
        go = torch.linspace(0.5, 2.0, N, device=dev).to(dt)
        go[::3] = 1.0
        loss.backward(go)
        exp = (g16.float() * go.float().cpu()[:, None]).to(dt)
    else:
        (loss * 3.0).backward()
        exp = (g16.float() * 3.0).to(dt)
    print(f"{name} autograd {reduction}", flush=True)
    assert zt.grad.dtype == dt
    assert torch.equal(zt.grad.cpu().view(torch.int16), exp.view(torch.int16))


def test_c_abi_typed(ext, dev):
    z16, y = case(1000, 256, 12, torch.bfloat16)
    zt, yt = z16.to(dev), torch.from_numpy(y).to(dev)
    out = fwloss_capi.forward_backward_typed(zt, yt)
    torch.cuda.synchronize()
    ref, g16 = expected(z16, y, 1.0 / 256)
    np.testing.assert_array_equal(out["kappa"].cpu().numpy(), ref["kappa"])
    assert torch.equal(out["grad"].cpu().view(torch.int16), g16.view(torch.int16))


@pytest.fixture
def reset_params16(ext):
    yield
    ext.set_params(0, 512)


@pytest.mark.parametrize("name", sorted(DTYPES))
@pytest.mark.parametrize("C,off", [(1000, 0), (1000, 8), (504, 24), (2000, 0), (8, 0)])
def test_dtype_offset_rows(ext, dev, name, C, off):
    """16-bit rows of 128-bit units starting `off` elements into a 128-byte line (logits and
    gradient alike), through path 1 and path 8 (16-bit rows keep plain addressing on both): the
    oracle's values bit-for-bit, and the elements around the gradient rows stay untouched."""
    N, pad = 300, 64
    z16, y = case(C, N, C + off, DTYPES[name])
    y[:2] = [0, C - 1]
    zbuf = torch.zeros(N * C + pad, dtype=z16.dtype, device=dev)
    zbuf[off:off + N * C] = z16.reshape(-1).to(dev)
    zt = zbuf[off:off + N * C].view(N, C)
    yt = torch.from_numpy(y).to(dev)
    ref, g16 = expected(z16, y, 1.0 / N)
    grads = []
    try:
        for path in (1, 8):
            ext.set_params(path, 512)
            gbuf = torch.full((N * C + pad,), 3.0, dtype=z16.dtype, device=dev)
            out = fwloss_capi.forward_backward_typed(zt, yt, grad=gbuf[off:off + N * C].view(N, C))
            torch.cuda.synchronize()
            g = gbuf.cpu()
            assert bool((g[:off] == 3.0).all()) and bool((g[off + N * C:] == 3.0).all())
            np.testing.assert_array_equal(out["kappa"].cpu().numpy(), ref["kappa"])
            np.testing.assert_array_equal(out["H"].cpu().numpy().view(np.uint32), ref["H"].view(np.uint32))
            np.testing.assert_array_equal(out["loss"].cpu().numpy().view(np.uint32), ref["loss"].view(np.uint32))
            grads.append(out["grad"].cpu())
            assert torch.equal(grads[-1].view(torch.int16), g16.view(torch.int16))
    finally:
        ext.set_params(0, 512)
