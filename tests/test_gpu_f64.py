"""float64 logits on the GPU (the reference CPU path's second dtype, src/cpu/fw_cpu.cpp:697-703).

Bar: against the compiled reference's float64 path (golden_f64.npz) and the fp64 definition oracle
(pinned to that reference and to exact rational arithmetic): kappa and the support equal, hence the
gradient bit-identical (scale / kappa on the support, minus scale at the label); tau and the losses
within 1e-14 relative (sums in a different fixed order); the mean within 1e-14.
"""
import os

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def run(ext, dev, z, y, scale=None, rdiv=None):
    N = z.shape[0]
    scale = (1.0 / N if N else 1.0) if scale is None else scale
    rdiv = float(N) if rdiv is None else rdiv
    H, loss, mean, kappa, grad = ext.fw_forward_backward(torch.from_numpy(z).to(dev), torch.from_numpy(y).to(dev),
                                                         scale, rdiv)
    assert H.dtype == loss.dtype == mean.dtype == grad.dtype == torch.float64
    return dict(H=H.cpu().numpy(), loss=loss.cpu().numpy(), mean=float(mean.cpu()), kappa=kappa.cpu().numpy(),
                grad=grad.cpu().numpy())


def check(out, ref, rtol=1e-14):
    bad = np.nonzero(out["kappa"] != ref["kappa"])[0]
    assert bad.size == 0, f"kappa differs on rows {bad[:10]}"
    np.testing.assert_allclose(out["H"], ref["tau"], rtol=rtol, atol=rtol)
    np.testing.assert_allclose(out["loss"], ref["loss"], rtol=rtol, atol=rtol)
    np.testing.assert_array_equal(out["grad"], ref["grad"])


@pytest.mark.parametrize("name", ["gauss", "ties", "wide", "flat"])
def test_reference_golden_vectors(ext, dev, name):
    g = np.load(os.path.join(HERE, "golden", "golden_f64.npz"))
    z, y, scale = g[f"{name}_z"], g[f"{name}_y"], float(g[f"{name}_scale"])
    out = run(ext, dev, z, y, scale)
    np.testing.assert_array_equal(out["kappa"], g[f"{name}_kappa"])
    np.testing.assert_allclose(out["loss"], g[f"{name}_L"], rtol=1e-14, atol=1e-14)
    G = np.zeros_like(z)
    G[g[f"{name}_g_rows"], g[f"{name}_g_cols"]] = g[f"{name}_g_vals"]
    np.testing.assert_array_equal(out["grad"], G)


@pytest.mark.parametrize("C", [1, 2, 7, 64, 100, 1000, 1001, 5000, 20001])
@pytest.mark.parametrize("kind", ["gauss", "ties", "tiny"])
def test_against_oracle(ext, dev, C, kind):
    rng = np.random.default_rng(C * 3 + len(kind))
    N = 300 if C <= 5000 else 40
    if kind == "gauss":
        z = rng.standard_normal((N, C)) * 2.0
    elif kind == "ties":
        z = 0.5 * rng.integers(-8, 9, (N, C)).astype(np.float64)
    else:
        z = rng.standard_normal((N, C)) * 1e-3      # every entry within 1 of the max: long supports
    y = rng.integers(0, C, N).astype(np.int64)
    out = run(ext, dev, z, y)
    ref = oracle.definition_f64(z, y)
    check(out, ref)
    assert abs(out["mean"] - ref["mean"]) <= 1e-14 * max(1.0, abs(ref["mean"]))


def test_long_supports_run_on_the_whole_row(ext, dev):
    """More than 512 candidates above the bound: the fixed-point iterations stream the row."""
    rng = np.random.default_rng(3)
    z = np.concatenate([np.zeros((4, 3000)), rng.standard_normal((4, 3000)) * 1e-4,
                        np.tile(np.linspace(0, 0.5, 3000), (4, 1))])
    y = rng.integers(0, 3000, z.shape[0]).astype(np.int64)
    out = run(ext, dev, z, y, 1.0, 1.0)
    ref = oracle.definition_f64(z, y, 1.0)
    check(out, ref, rtol=1e-13)
    assert (out["kappa"][:4] == 3000).all()


def test_special_values(ext, dev):
    C = 50
    rng = np.random.default_rng(8)
    z = rng.standard_normal((6, C))
    z[0, :10] = -np.inf                      # -inf entries are never selected
    z[1, 3] = -np.inf
    z[2, 5] = -0.0
    z[2, 6] = 0.0
    z[3, 7] = np.nan                         # NaN entries are never selected
    y = rng.integers(0, C, 6).astype(np.int64)
    y[0] = 11
    y[1] = 3                                 # label at -inf: loss +inf
    out = run(ext, dev, z, y, 1.0, 1.0)
    fin = np.where(np.isnan(z), -np.inf, z)
    ref = oracle.definition_f64(fin, y, 1.0)
    np.testing.assert_array_equal(out["kappa"], ref["kappa"])
    np.testing.assert_allclose(out["H"], ref["tau"], rtol=1e-14)
    assert np.isposinf(out["loss"][1])
    np.testing.assert_array_equal(out["grad"], ref["grad"])


def test_rows_without_a_finite_maximum(ext, dev):
    z = np.full((3, 8), -np.inf)
    z[1, :] = np.nan
    z[2, 2] = np.inf
    y = np.array([1, 2, 3], np.int64)
    out = run(ext, dev, z, y, 1.0, 1.0)
    assert (out["kappa"] == 0).all() and np.isnan(out["H"]).all() and np.isnan(out["loss"]).all()
    g = np.zeros_like(z)
    g[np.arange(3), y] = -1.0
    np.testing.assert_array_equal(out["grad"], g)


def test_bad_labels_and_empty_batch(ext, dev):
    z = np.random.default_rng(2).standard_normal((4, 9))
    y = np.array([0, -1, 9, 4], np.int64)
    out = run(ext, dev, z, y, 1.0, 1.0)
    assert np.isnan(out["loss"][1]) and np.isnan(out["loss"][2])
    ref = oracle.definition_f64(z, np.array([0, 0, 0, 4], np.int64), 1.0)
    np.testing.assert_array_equal(out["kappa"], ref["kappa"])
    g = ref["grad"].copy()
    g[1, 0] += 1.0
    g[2, 0] += 1.0                           # no label term on the rows with a bad label
    np.testing.assert_array_equal(out["grad"], g)
    e = run(ext, dev, np.zeros((0, 5)), np.zeros(0, np.int64))
    assert e["grad"].shape == (0, 5)


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_autograd(ext, dev, reduction):
    rng = np.random.default_rng(4)
    N, C = 200, 777
    z = rng.standard_normal((N, C)) * 1.5
    y = rng.integers(0, C, N).astype(np.int64)
    zt = torch.from_numpy(z).to(dev).requires_grad_(True)
    loss = ext.familywise_loss(zt, torch.from_numpy(y).to(dev), reduction)
    assert loss.dtype == torch.float64
    ref = oracle.definition_f64(z, y, 1.0)
    if reduction == "none":
        go = rng.uniform(-2, 2, N)
        loss.backward(torch.from_numpy(go).to(dev))
        np.testing.assert_allclose(loss.detach().cpu().numpy(), ref["loss"], rtol=1e-14)
        want = ref["grad"] * go[:, None]
    else:
        loss.backward()
        s = 1.0 / N if reduction == "mean" else 1.0
        total = ref["loss"].sum() * s
        assert abs(loss.item() - total) <= 1e-13 * max(1.0, abs(total))
        want = oracle.definition_f64(z, y, s)["grad"]
    np.testing.assert_allclose(zt.grad.cpu().numpy(), want, rtol=1e-15, atol=0)


def test_fw_loss_grad_float64(ext, dev):
    rng = np.random.default_rng(6)
    z = rng.standard_normal((64, 300))
    y = rng.integers(0, 300, 64).astype(np.int64)
    L, G, k = ext.fw_loss_grad(torch.from_numpy(z).to(dev), torch.from_numpy(y).to(dev), 0.5)
    ref = oracle.definition_f64(z, y, 0.5)
    assert L.dtype == torch.float64 and G.dtype == torch.float64 and k.dtype == torch.int64
    np.testing.assert_allclose(L.cpu().numpy(), ref["loss"], rtol=1e-14)
    np.testing.assert_array_equal(G.cpu().numpy(), ref["grad"])


@pytest.mark.parametrize("C", [1000, 5001])
def test_graph_capture_replays(ext, dev, C):
    """The float64 path allocates nothing and records no memset: a captured call replays to the
    eager result, with eager work between the replays (register rows and streamed rows)."""
    rng = np.random.default_rng(C)
    z = torch.from_numpy(rng.standard_normal((300, C))).to(dev)
    y = torch.from_numpy(rng.integers(0, C, 300).astype(np.int64)).to(dev)
    eager = ext.fw_forward_backward(z, y)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ext.fw_forward_backward(z, y)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ext.fw_forward_backward(z, y)
    print(f"f64 graph replays C={C}", flush=True)
    for it in range(4):
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(out, eager):
            assert torch.equal(a, b), f"replay {it} differs from the eager result"
        _ = ext.fw_forward_backward(z, y)
        torch.cuda.synchronize()
