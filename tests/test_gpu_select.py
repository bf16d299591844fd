"""The bounded threshold select and the call-level contract of the fused op.

* Rows whose candidates within 1 of the maximum outnumber the LDS lists: the low-sigma inputs of the
  reference's GPU harness (Gaussian, Laplace and 50/50 mixture logits swept over sigma,
  benchmarks/cuda_benchmarks/data_io.py:8-83, CE_FW_perf.py:94-96).  The register kernel bounds
  them from the tau of its 64 lane maxima; the streaming kernels tighten their lists with the
  round in registers, and rows that still overflow are solved in memory (histogram passes,
  refinements, a collect pass; a bisection as the last resort).  Every result is checked against the
  oracle: bit-exact kappa, H, losses and gradient on reduced batches, size-independent properties
  at full size.
* Per-call options from several host threads at once, a workspace with any contents, logits read
  at a row stride, the fp64 per-row losses against the compiled reference's golden values, guard
  bands after the last row, a second backward, and graph replays after the workspace grew.
"""
import ctypes
import os
import threading

import numpy as np
import pytest
import torch

import fwloss_capi
import fwloss_data as data
import oracle
from test_gpu_parity import _row_properties, assert_parity, bits_equal, fused, to_dev

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture
def reset_params(ext):
    yield
    ext.set_params(0, 512)


# rows per reduced batch: enough rows for every kernel family at that length (the split kernels
# take <= 128 rows of >= 96 KiB, the overflow kernel follows the streaming ones)
REDUCED_ROWS = {1000: 512, 8192: 96, 32000: 40, 131072: 12}


@pytest.mark.parametrize("C", sorted(REDUCED_ROWS))
@pytest.mark.parametrize("sigma", [0.001, 0.01, 100.0])
@pytest.mark.parametrize("dist", ["gauss", "laplace"])
def test_dist_parity(ext, dev, dist, sigma, C):
    z, y = data.make_dist(dist, REDUCED_ROWS[C], C, sigma, seed=3)
    print(f"dist {dist} sigma={sigma} N={z.shape[0]} C={C}", flush=True)
    ref = oracle.definition(z, y)
    assert_parity(fused(ext, *to_dev(dev, z, y)), ref, z)


@pytest.mark.parametrize("C", [1000, 8192, 32000])
@pytest.mark.parametrize("sigma", [0.001, 0.01])
def test_mixture_parity(ext, dev, sigma, C):
    z, y = data.make_dist("mixture", REDUCED_ROWS[C], C, sigma, seed=4)
    print(f"mixture sigma={sigma} C={C}", flush=True)
    assert_parity(fused(ext, *to_dev(dev, z, y)), oracle.definition(z, y), z)


@pytest.mark.parametrize("N,C", [(160, 131072), (400, 32000), (700, 8192), (3000, 3000)])
def test_dist_overflow_kernel(ext, dev, N, C):
    """Enough rows for the streaming kernels (not the split ones): every low-sigma row overflows
    its list and is solved by the overflow kernel; other rows stay on the list path."""
    z, y = data.make_dist("gauss", N, C, 1.0, seed=5)
    z[::3] *= np.float32(0.001)
    z[1::3] *= np.float32(0.01)
    print(f"overflow kernel N={N} C={C}", flush=True)
    ref = oracle.definition(z, y)
    assert_parity(fused(ext, *to_dev(dev, z, y)), ref, z)


@pytest.mark.parametrize("C", [5000, 40000])
def test_dist_drop_in_ops(ext, dev, C):
    """The mask and candidate-list forwards on low-sigma rows (the overflow kernel writes the mask
    and the whole support list)."""
    N = 300
    z, y = data.make_dist("gauss", N, C, 0.001, seed=6)
    z[::4] = np.random.default_rng(1).standard_normal((len(z[::4]), C)).astype(np.float32)
    zt, yt = to_dev(dev, z, y)
    ref = oracle.definition(z, y)
    print(f"drop-in small C={C}", flush=True)
    H, loss, mean, kappa, sel = ext.fw_forward_small(zt, yt)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(kappa.cpu().numpy(), ref["kappa"])
    assert bits_equal(H.cpu().numpy(), ref["H"])
    np.testing.assert_array_equal(sel.cpu().numpy(), z > ref["tau"][:, None])
    print(f"drop-in large C={C}", flush=True)
    H, loss, mean, kappa, cb, ci, cc = ext.fw_forward(zt, yt)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(cc.cpu().numpy(), ref["kappa"])
    ci, cb = ci.cpu().numpy(), cb.cpu().numpy()
    for r in range(0, N, 7):
        k = int(ref["kappa"][r])
        idx = ci[r, :k]
        assert np.array_equal(np.sort(idx), np.nonzero(z[r] > ref["tau"][r])[0]), f"row {r}"
        np.testing.assert_array_equal(cb[r, :k], z[r, idx])
    g = ext.fw_backward(zt, yt, H, kappa, torch.from_numpy(cb).to(dev), torch.from_numpy(ci).to(dev), cc)
    torch.cuda.synchronize()
    assert bits_equal(g.cpu().numpy(), ref["grad"])


def ties_rows(N, C, seed):
    """Rows whose boundary falls among many equal values: dyadic ties, constant rows, two levels."""
    rng = np.random.default_rng(seed)
    z = (0.5 * rng.integers(-2, 3, (N, C))).astype(np.float32)
    z[1::4] = np.float32(rng.standard_normal())
    half = rng.random((len(z[2::4]), C)) < 0.5
    z[2::4] = np.where(half, np.float32(1.0), np.float32(0.999)).astype(np.float32)
    z[3::4] *= np.float32(1e-3)
    return z, rng.integers(0, C, N)


@pytest.mark.parametrize("path", [3, 5])
@pytest.mark.parametrize("cap", [64, 512])
@pytest.mark.parametrize("C", [100, 3000, 20000])
def test_forced_overflow_solve(ext, dev, reset_params, path, cap, C):
    """Every row through the overflow solve (paths 3, 5), with small lists (cap 64: collect lists of
    128/512 entries) so that dense bins take the key refinements, down to single keys."""
    z, y = ties_rows(24, C, seed=C)
    z2, y2 = data.make_dist("laplace", 24, C, 0.001, seed=C)
    z, y = np.concatenate([z, z2]), np.concatenate([y, y2])
    ext.set_params(path, cap)
    print(f"forced path={path} cap={cap} C={C}", flush=True)
    assert_parity(fused(ext, *to_dev(dev, z, y)), oracle.definition(z, y), z)


@pytest.mark.parametrize("C", [5000, 40000])
def test_no_workspace_overflow(ext, dev, C):
    """Without a workspace the streaming kernels solve overflowing rows themselves (bisection)."""
    N = 64
    z, y = data.make_dist("gauss", N, C, 0.001, seed=7)
    zt, yt = to_dev(dev, z, y)
    ref = oracle.definition(z, y)
    L = fwloss_capi.lib()
    H = torch.empty(N, device=dev)
    loss = torch.empty(N, device=dev)
    kappa = torch.empty(N, dtype=torch.int32, device=dev)
    grad = torch.empty_like(zt)
    P = ctypes.c_void_p
    print(f"no workspace C={C}", flush=True)
    rc = L.fwl_forward_backward(P(zt.data_ptr()), P(yt.data_ptr()), N, C, 1.0 / N, float(N), P(H.data_ptr()),
                                P(loss.data_ptr()), None, P(kappa.data_ptr()), P(grad.data_ptr()), None, 0,
                                P(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    assert_parity(dict(H=H.cpu().numpy(), loss=loss.cpu().numpy(), kappa=kappa.cpu().numpy(),
                       grad=grad.cpu().numpy()), ref, z)


@pytest.mark.parametrize("dist,shape", [("gauss", (65536, 1000)), ("laplace", (65536, 1000)),
                                        ("gauss", (2048, 131072)), ("laplace", (8192, 32000))])
def test_dist_full_size(ext, dev, dist, shape):
    N, C = shape
    z, y = data.make_dist(dist, N, C, 0.001, seed=0)
    print(f"full size {dist} sigma=0.001 N={N} C={C}", flush=True)
    zt, yt = to_dev(dev, z, y)
    H, loss, mean, kappa, grad = ext.fw_forward_backward(zt, yt)
    torch.cuda.synchronize()
    _row_properties(zt, yt, H, loss, kappa, grad, 1.0 / N)
    assert abs(mean.item() - loss.double().mean().item()) <= 1e-6 * max(1.0, abs(mean.item()))
    rows = np.random.default_rng(0).choice(N, size=32, replace=False)
    ref = oracle.definition(z[rows], y[rows], scale=1.0 / N)
    sub = dict(H=H[rows].cpu().numpy(), loss=loss[rows].cpu().numpy(), kappa=kappa[rows].cpu().numpy(),
               grad=grad[rows].cpu().numpy(), mean=None)
    assert_parity(sub, ref, z[rows])
    del zt, grad
    torch.cuda.empty_cache()


# ---------------------------------------------------------------- the two-pass op's write pass

def list_mix(N, C, seed):
    """Rows for the two-pass op: N(0, sigma) rows over sigma (supports from a handful of entries to
    most of the row), ascending rows (every element is a candidate), constant rows and dyadic
    ties."""
    rng = np.random.default_rng(seed)
    z, y = data.make_dist("gauss", N, C, 1.0, seed=seed)
    sig = np.array([1.0, 0.1, 0.01, 0.001, 5e-4, 1e-4, 100.0, 1.0], np.float32)
    z *= sig[np.arange(N) % len(sig)][:, None]
    z[8::32] = np.sort(z[8::32], axis=1)
    z[9::32] = np.float32(0.25)
    z[10::32] = (0.5 * rng.integers(-2, 3, (len(z[10::32]), C))).astype(np.float32)
    return z, y


@pytest.mark.parametrize("path", [2, 3])
@pytest.mark.parametrize("C", [4096, 4099, 20000])
def test_two_pass_lists(ext, dev, reset_params, path, C):
    """2048 rows through the forced two-pass paths.  Rows of whole 128-bit units (C = 4096, 20000)
    take the 4 KB-block write pass: zeros for rows whose support the read pass listed (at most 512
    entries, from a list that kept its indices; the scatter kernel adds them), the others from the
    logits.  C = 4099 takes the fill and scatter kernels.  Path 3 sends every row through the
    overflow solve.  The rows cover supports of a few, of 65-512 and of more than 512 entries."""
    z, y = list_mix(2048, C, seed=C + path)
    ext.set_params(path, 512)
    print(f"two-pass lists path={path} C={C}", flush=True)
    ref = oracle.definition(z, y)
    k = ref["kappa"]
    assert (k <= 64).any() and ((k > 64) & (k <= 512)).any() and (k > 512).any()
    assert_parity(fused(ext, *to_dev(dev, z, y)), ref, z)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_two_pass_odd_16bit_windows(ext, dev, reset_params, dtype):
    """16-bit rows of odd length, long and many (2048 x 32001): the default dispatch takes the
    two-pass op, whose read pass streams every row through a window from the 4-byte boundary below
    it with 128-bit loads (the element in front of the row masked, the last dword whole)."""
    z, y = list_mix(2048, 32001, seed=11)
    z16 = torch.from_numpy(z).to(dtype)
    z32 = z16.float().numpy()
    ref = oracle.definition(z32, y)
    ext.set_params(0, 512)
    print(f"two-pass odd 16-bit windows {dtype}", flush=True)
    H, loss, mean, kappa, grad = ext.fw_forward_backward(z16.to(dev), torch.from_numpy(y).to(dev))
    torch.cuda.synchronize()
    assert_parity(dict(H=H.cpu().numpy(), loss=loss.cpu().numpy(), kappa=kappa.cpu().numpy(), mean=float(mean.cpu())),
                  ref, z32)
    g16 = torch.from_numpy(ref["grad"]).to(dtype)
    assert torch.equal(grad.cpu().view(torch.int16), g16.view(torch.int16)), "grad not bit-identical"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("path", [2, 3])
@pytest.mark.parametrize("C", [4096, 4097])
def test_two_pass_lists_16bit(ext, dev, reset_params, dtype, path, C):
    """The same in 16-bit logits: rows of whole 128-bit units (the 4 KB-block write pass) and odd
    rows (the fill and scatter kernels)."""
    z, y = list_mix(2048, C, seed=C + 7 * path)
    z16 = torch.from_numpy(z).to(dtype)
    z32 = z16.float().numpy()
    ref = oracle.definition(z32, y)
    ext.set_params(path, 512)
    print(f"two-pass lists {dtype} path={path} C={C}", flush=True)
    H, loss, mean, kappa, grad = ext.fw_forward_backward(z16.to(dev), torch.from_numpy(y).to(dev))
    torch.cuda.synchronize()
    assert_parity(dict(H=H.cpu().numpy(), loss=loss.cpu().numpy(), kappa=kappa.cpu().numpy(), mean=float(mean.cpu())),
                  ref, z32)
    g16 = torch.from_numpy(ref["grad"]).to(dtype)
    assert torch.equal(grad.cpu().view(torch.int16), g16.view(torch.int16)), "grad not bit-identical"


# ---------------------------------------------------------------- the call-level contract

def test_per_call_options_from_threads(ext, dev):
    """Two host threads, each on its own stream, force different kernel families per call (the
    register kernel, the streaming kernel with small lists, the overflow solve); neither changes
    the other's dispatch, and every result is the oracle's."""
    rng = np.random.default_rng(9)
    z = rng.standard_normal((256, 3000)).astype(np.float32)
    z[::2] *= np.float32(0.002)
    y = rng.integers(0, 3000, 256)
    ref = oracle.definition(z, y)
    zt, yt = to_dev(dev, z, y)
    results, errors = {}, []

    def work(name, path, cap):
        try:
            s = torch.cuda.Stream(device=dev)
            with torch.cuda.stream(s):
                outs = []
                for _ in range(6):
                    H, loss, mean, kappa, grad = ext.fw_forward_backward(zt, yt, path=path, cand_cap=cap)
                    outs.append((H, loss, mean, kappa, grad))
            s.synchronize()
            results[name] = [dict(H=o[0].cpu().numpy(), loss=o[1].cpu().numpy(), mean=float(o[2].cpu()),
                                  kappa=o[3].cpu().numpy(), grad=o[4].cpu().numpy()) for o in outs]
        except Exception as e:   # reported by the main thread
            errors.append(e)
    threads = [threading.Thread(target=work, args=("wave", 4, 64)), threading.Thread(target=work, args=("solve", 5, 512)),
               threading.Thread(target=work, args=("block", 2, 64))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    assert tuple(ext.get_params()) == (0, 512)   # the process defaults are untouched
    for name, outs in results.items():
        for out in outs:
            assert_parity(out, ref, z)


def test_dirty_workspace(ext, dev):
    """The workspace holds no state between calls: filled with arbitrary bytes before every call,
    it still gives the oracle's results and the right mean (register, streaming and two-pass
    shapes, with and without overflowing rows)."""
    for (N, C, sigma) in [(2048, 1000, 1.0), (300, 3000, 0.001), (400, 32000, 1.0), (400, 32000, 0.001)]:
        z, y = data.make_dist("gauss", N, C, sigma, seed=N + C)
        zt, yt = to_dev(dev, z, y)
        ref = oracle.definition(z, y)
        ws = fwloss_capi.Workspace(dev)
        for fill in (0xFF, 0x7F, 0x00, 0xA5):
            buf = ws.get(N, C)
            buf.fill_(fill)
            print(f"dirty workspace N={N} C={C} sigma={sigma} fill={fill:#x}", flush=True)
            out = fwloss_capi.forward_backward(zt, yt, ws=ws)
            torch.cuda.synchronize()
            got = {k: (v.cpu().numpy() if v.dim() else float(v.cpu())) for k, v in out.items()}
            assert_parity(got, ref, z)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N,C,skip", [(64, 1000, 1), (64, 1000, 8), (40, 5000, 3), (400, 32000, 4), (8, 100, 5),
                                      (12, 40000, 1)])
def test_row_stride(ext, dev, dtype, N, C, skip):
    """Logits read in place at a row stride (a column slice of a wider tensor): the same results as
    on a contiguous copy, with no copy made (the op reads the view's storage)."""
    rng = np.random.default_rng(C + skip)
    wide = torch.from_numpy(rng.standard_normal((N, C + skip)).astype(np.float32)).to(dev).to(dtype)
    zt = wide[:, skip:]
    yt = torch.from_numpy(rng.integers(0, C, N)).to(dev)
    assert not zt.is_contiguous()
    z = zt.float().cpu().numpy()
    ref = oracle.definition(z, yt.cpu().numpy())
    print(f"row stride {dtype} N={N} C={C} skip={skip}", flush=True)
    H, loss, mean, kappa, grad = ext.fw_forward_backward(zt, yt)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(kappa.cpu().numpy(), ref["kappa"])
    assert bits_equal(H.cpu().numpy(), ref["H"])
    assert bits_equal(loss.cpu().numpy(), ref["loss"])
    expect = torch.from_numpy(ref["grad"]).to(dtype)
    assert torch.equal(grad.cpu(), expect)
    # the C ABI with the same stride
    out = fwloss_capi.forward_backward_ex(zt, yt)
    torch.cuda.synchronize()
    assert torch.equal(out["grad"].cpu(), expect)
    np.testing.assert_array_equal(out["kappa"].cpu().numpy(), ref["kappa"])


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3", "cfg4", "cfg5", "edges"])
def test_loss64_matches_golden(ext, dev, cfg):
    """fw_loss_grad's fp64 per-row losses against the compiled reference's fw_loss_grad L
    (src/cpu/fw_cpu.cpp:614, :750-757), golden vectors in tests/golden/, rtol 1e-12."""
    g = np.load(os.path.join(GOLDEN, f"golden_{cfg}.npz"))
    z, y = g["z"], g["y"]
    zt, yt = to_dev(dev, z, y)
    L, G, k = ext.fw_loss_grad(zt, yt, float(g["scale"]))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(k.cpu().numpy(), g["kappa"])
    Lr, Lg = g["L"], L.cpu().numpy()
    fin = np.isfinite(Lr)
    np.testing.assert_array_equal(np.isfinite(Lg), fin)
    # rows with |z| >= 2^53 lose the 1 of 1 - z_y in fp64: there the reference's evaluation order
    # (1 + (thr - z_y) + (tau - thr), fw_cpu.cpp:614) and (1 - z_y) + tau round differently (the
    # golden +-1e30 edge row: 1.2e-10 relative); every other row agrees to 1e-12
    huge = np.abs(z).max(axis=1) >= 2.0 ** 53
    np.testing.assert_allclose(Lg[fin & ~huge], Lr[fin & ~huge], rtol=1e-12, atol=0)
    np.testing.assert_allclose(Lg[fin & huge], Lr[fin & huge], rtol=1e-9, atol=0)


@pytest.mark.parametrize("path", [1, 4])
@pytest.mark.parametrize("dtype,C", [(torch.float32, 1001), (torch.float32, 1003), (torch.float32, 2047),
                                     (torch.bfloat16, 1002), (torch.float16, 1002)])
def test_guard_band_after_last_row(ext, dev, reset_params, path, dtype, C):
    """Rows whose last 128-bit unit runs past the row end rely on the per-dword range check of the
    buffer resource: the bytes after the last row's gradient stay untouched (register and
    streaming kernels), and every row matches the oracle."""
    N = 37
    rng = np.random.default_rng(C)
    z = rng.standard_normal((N, C)).astype(np.float32)
    y = rng.integers(0, C, N)
    zt = torch.from_numpy(z).to(dev).to(dtype)
    yt = torch.from_numpy(y).to(dev)
    pad = 256
    sentinel = {torch.float32: 1234.5, torch.bfloat16: 77.0, torch.float16: -3.5}[dtype]
    buf = torch.full((N * C + pad,), sentinel, dtype=dtype, device=dev)
    grad = buf[: N * C].view(N, C)
    ext.set_params(path, 512)
    print(f"guard band path={path} {dtype} C={C}", flush=True)
    fwloss_capi.forward_backward_typed(zt, yt, grad=grad)
    torch.cuda.synchronize()
    assert torch.all(buf[N * C:] == sentinel), "bytes after the last row were written"
    ref = oracle.definition(zt.float().cpu().numpy(), y)
    assert torch.equal(grad.cpu(), torch.from_numpy(ref["grad"]).to(dtype))


def test_second_backward_raises(ext, dev):
    z, y = data.make("cfg2", N=64, seed=2)
    zt, yt = to_dev(dev, z, y)
    zt.requires_grad_(True)
    loss = ext.familywise_loss(zt, yt)
    (loss * 2.0).backward(retain_graph=True)
    g1 = zt.grad.clone()
    with pytest.raises(RuntimeError, match="already ran"):
        (loss * 2.0).backward()
    assert torch.equal(zt.grad, g1)   # nothing accumulated by the refused call


def test_graph_replay_after_workspace_growth(ext, dev):
    """A graph captured with the stream's workspace keeps working after a larger call on the same
    stream grew the workspace, and after other tensors took freed memory: the superseded workspace
    stays allocated."""
    s = torch.cuda.Stream(device=dev)
    z, y = data.make("cfg2", N=512, seed=31)
    zt, yt = to_dev(dev, z, y)
    ref = oracle.definition(z, y)
    with torch.cuda.stream(s):
        for _ in range(2):
            ext.fw_forward_backward(zt, yt)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = ext.fw_forward_backward(zt, yt)
    # a larger call on the same stream grows its workspace
    zb, yb = data.make_dist("gauss", 3000, 40000, 0.001, seed=1)
    zbt, ybt = to_dev(dev, zb, yb)
    with torch.cuda.stream(s):
        big = ext.fw_forward_backward(zbt, ybt)
    s.synchronize()
    del big, zbt, ybt
    torch.cuda.empty_cache()
    junk = [torch.full((1 << 20,), 7.0, device=dev) for _ in range(64)]
    for _ in range(3):
        g.replay()
        s.synchronize()
        got = dict(H=outs[0].cpu().numpy(), loss=outs[1].cpu().numpy(), mean=float(outs[2].cpu()),
                   kappa=outs[3].cpu().numpy(), grad=outs[4].cpu().numpy())
        assert_parity(got, ref, z)
        assert all(bool(torch.all(j == 7.0)) for j in junk)
