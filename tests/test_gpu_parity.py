"""Parity of the HIP path with the CPU oracle (the definition, reference_impl.py:11-35, with the
strict-support semantics of src/cpu/fw_cpu.cpp:96-101).

Bar: kappa, the support (mask / candidate lists), H, per-row losses and the gradient are
bit-identical to the oracle on every seeded configuration; the mean loss is within 1e-6 relative
(it is summed in a different fixed order).  Full-size configurations are checked through
size-independent properties plus a random sample of rows against the oracle.
"""
import numpy as np
import pytest
import torch

import fwloss_capi
import fwloss_data as data
import oracle

pytestmark = pytest.mark.gpu


def to_dev(dev, z, y):
    return torch.from_numpy(z).to(dev), torch.from_numpy(y).to(dev)


def fused(ext, zt, yt, scale=-1.0, rdiv=-1.0):
    H, loss, mean, kappa, grad = ext.fw_forward_backward(zt, yt, scale, rdiv)
    torch.cuda.synchronize()
    return dict(H=H.cpu().numpy(), loss=loss.cpu().numpy(), mean=float(mean.cpu()),
                kappa=kappa.cpu().numpy(), grad=grad.cpu().numpy())


def bits_equal(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    if a.shape != b.shape:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def assert_parity(out, ref, z, mean_rtol=1e-6):
    bad = np.nonzero(out["kappa"] != ref["kappa"])[0]
    assert bad.size == 0, f"kappa differs on rows {bad[:10]}: {out['kappa'][bad[:10]]} vs {ref['kappa'][bad[:10]]}"
    assert bits_equal(out["H"], ref["H"]), "H not bit-identical"
    assert bits_equal(out["loss"], ref["loss"]), "losses not bit-identical"
    if "grad" in out:
        assert bits_equal(out["grad"], ref["grad"]), "grad not bit-identical"
    if out.get("mean") is not None and z.shape[0] > 0 and np.isfinite(ref["mean"]):
        assert abs(out["mean"] - ref["mean"]) <= mean_rtol * max(1.0, abs(ref["mean"]))


@pytest.fixture
def reset_params(ext):
    yield
    ext.set_params(0, 512)


# ---------------------------------------------------------------- seeded configurations (reduced N)

REDUCED = {"cfg1": 1024, "cfg2": 2048, "cfg3": 16384, "cfg4": 96, "cfg5": 24, "mid3000": 256, "mid2999": 256}


def make_case(name, N, seed):
    """A seeded configuration, or "mid<C>": mid-range C rows (N(0,1), every 5th row flat)."""
    if name.startswith("mid"):
        C = int(name[3:])
        rng = np.random.default_rng(seed)
        z = rng.standard_normal((N, C)).astype(np.float32)
        z[::5] *= np.float32(0.02)
        return z, rng.integers(0, C, N)
    return data.make(name, N=N, seed=seed)


@pytest.mark.parametrize("cfg", sorted(REDUCED))
def test_fused_matches_oracle(ext, dev, cfg):
    z, y = make_case(cfg, REDUCED[cfg], 1)
    print(f"fused {cfg} N={z.shape[0]} C={z.shape[1]}", flush=True)
    ref = oracle.definition(z, y)
    out = fused(ext, *to_dev(dev, z, y))
    assert_parity(out, ref, z)


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3", "cfg4", "mid3000", "mid2999"])
def test_drop_in_small_ops(ext, dev, cfg):
    z, y = make_case(cfg, min(REDUCED[cfg], 512), 2)
    print(f"small ops {cfg} N={z.shape[0]}", flush=True)
    zt, yt = to_dev(dev, z, y)
    H, losses, mean, kappa, sel = ext.fw_forward_small(zt, yt)
    grad = ext.fw_backward_small(yt, sel, kappa)
    torch.cuda.synchronize()
    ref = oracle.definition(z, y)
    assert sel.dtype == torch.bool and sel.shape == zt.shape
    assert kappa.dtype == torch.int32 and mean.dim() == 0
    np.testing.assert_array_equal(sel.cpu().numpy(), z > ref["tau"][:, None])
    out = dict(H=H.cpu().numpy(), loss=losses.cpu().numpy(), mean=float(mean.cpu()), kappa=kappa.cpu().numpy(),
               grad=grad.cpu().numpy())
    assert_parity(out, ref, z)


@pytest.mark.parametrize("cfg", ["cfg2", "cfg3", "cfg4", "cfg5", "mid3000", "mid2999"])
def test_drop_in_large_ops(ext, dev, cfg):
    z, y = make_case(cfg, min(REDUCED[cfg], 256), 3)
    print(f"large ops {cfg} N={z.shape[0]}", flush=True)
    zt, yt = to_dev(dev, z, y)
    H, losses, mean, kappa, cbuf, cidx, ccnt = ext.fw_forward(zt, yt)
    grad = ext.fw_backward(zt, yt, H, kappa, cbuf, cidx, ccnt)
    torch.cuda.synchronize()
    ref = oracle.definition(z, y)
    cnt = ccnt.cpu().numpy()
    np.testing.assert_array_equal(cnt, ref["kappa"])
    cb, ci = cbuf.cpu().numpy(), cidx.cpu().numpy()
    for r in range(z.shape[0]):
        idx = ci[r, :cnt[r]]
        assert np.array_equal(np.sort(idx), np.nonzero(z[r] > ref["tau"][r])[0]), f"row {r} support"
        assert bits_equal(cb[r, :cnt[r]], z[r, idx])
    out = dict(H=H.cpu().numpy(), loss=losses.cpu().numpy(), mean=float(mean.cpu()), kappa=kappa.cpu().numpy(),
               grad=grad.cpu().numpy())
    assert_parity(out, ref, z)


# ---------------------------------------------------------------- every kernel path, same answers

@pytest.mark.parametrize("path,cap", [(1, 512), (2, 512), (2, 64), (3, 512), (4, 512), (4, 64), (5, 512), (6, 512)])
@pytest.mark.parametrize("C", [10, 64, 100, 256, 1000, 1024, 2999, 3000])
def test_forced_paths(ext, dev, reset_params, path, cap, C):
    rng = np.random.default_rng(C)
    z = rng.standard_normal((300, C)).astype(np.float32)
    z[::7] *= np.float32(0.01)          # flat rows: many candidates, long supports
    z[3::11] = np.round(z[3::11] * 2) / 2   # dyadic ties
    y = rng.integers(0, C, 300)
    print(f"path={path} cap={cap} C={C}", flush=True)
    ext.set_params(path, cap)
    ref = oracle.definition(z, y)
    out = fused(ext, *to_dev(dev, z, y))
    assert_parity(out, ref, z)


@pytest.mark.parametrize("path", [2, 4])
@pytest.mark.parametrize("cap", [64, 512])
def test_streamed_overflow_and_tighten(ext, dev, reset_params, path, cap):
    # C = 4096 rows: a flat row overflows any list (generic path), a row with many candidates but a
    # short support exercises list tightening
    rng = np.random.default_rng(7)
    C = 4096
    z = rng.standard_normal((64, C)).astype(np.float32)
    z[0] = 0.0
    z[1] = rng.random(C).astype(np.float32) * np.float32(0.9)       # all candidates, short support
    z[2, :] = np.float32(1e-3) * rng.standard_normal(C).astype(np.float32)
    z[3, ::2] = 5.0
    y = rng.integers(0, C, 64)
    print(f"streamed overflow path={path} cap={cap}", flush=True)
    ext.set_params(path, cap)
    ref = oracle.definition(z, y)
    assert_parity(fused(ext, *to_dev(dev, z, y)), ref, z)


# ---------------------------------------------------------------- split rows: few long rows

def _split_case(N, C, seed):
    rng = np.random.default_rng(seed)
    z = (rng.standard_normal((N, C)) * rng.choice([0.05, 1.0, 4.0], size=(N, 1))).astype(np.float32)
    z[::7] *= np.float32(0.01)                   # flat rows: long chunk supports (generic solve)
    z[3::11] = np.round(z[3::11] * 2) / 2        # dyadic ties
    z[5::13, -1] = z[5::13].max(axis=1) + 3      # the maximum in the last (possibly short) chunk
    y = rng.integers(0, C, N)
    return z, y


@pytest.mark.parametrize("N,C", [(1, 1), (3, 10), (5, 1000), (16, 1024), (7, 2999), (128, 3000), (33, 20000),
                                 (2, 70001), (128, 4097), (300, 3000)])
def test_split_rows_forced(ext, dev, reset_params, N, C):
    # path 7 at any length: one chunk, a short last chunk, up to 256 chunks per row (300 rows:
    # beyond path 7's 128, so one block per row runs)
    z, y = _split_case(N, C, N * 7 + C)
    print(f"split forced N={N} C={C}", flush=True)
    ext.set_params(7, 512)
    assert_parity(fused(ext, *to_dev(dev, z, y)), oracle.definition(z, y), z)


@pytest.mark.parametrize("N,C", [(1, 24575), (1, 24576), (16, 50000), (3, 131072), (128, 32000), (129, 24576)])
def test_split_rows_auto(ext, dev, N, C):
    # the automatic rule: rows of >= 96 KiB (24576 fp32 elements), at most 128 of them; the
    # shapes just outside it (24575 elements, 129 rows) run one block per row
    z, y = _split_case(N, C, N + C)
    print(f"split auto N={N} C={C}", flush=True)
    assert_parity(fused(ext, *to_dev(dev, z, y)), oracle.definition(z, y), z)


def test_split_rows_union_sizes(ext, dev, reset_params):
    # 40 chunks of 1024 per row, a plateau of near-equal values in every chunk: per chunk 20, 40 or
    # 60 support entries (kept), or 70 (too many to keep: generic solve); the union of the kept
    # entries has 800 (a long list for the finishing wavefront), 1600 or 2400 (generic) entries
    rng = np.random.default_rng(3)
    C = 40960
    per = [20, 40, 60, 70, 20, 5]
    z = np.full((len(per), C), -5.0, np.float32)
    z += np.float32(1e-3) * rng.standard_normal(z.shape).astype(np.float32)
    for r, k in enumerate(per):
        for c in range(40):
            pos = c * 1024 + rng.choice(1024, k, replace=False)
            z[r, pos] = np.float32(1.0) + np.float32(1e-3) * rng.standard_normal(k).astype(np.float32)
    z[4, 1024:2048] = -np.inf                    # a chunk with no finite entry
    z[5, 3 * 1024:] = -np.inf                    # only 3 chunks with finite entries
    y = rng.integers(0, C, len(per))
    y[5] = C - 1                                 # label at -inf
    ref = oracle.definition(z, y)
    for path in (7, 0):
        print(f"split union sizes path={path}", flush=True)
        ext.set_params(path, 512)
        assert_parity(fused(ext, *to_dev(dev, z, y)), ref, z)


@pytest.mark.parametrize("C", [5000, 40000])
def test_split_rows_drop_in_ops(ext, dev, reset_params, C):
    # support mask and candidate-list outputs of the split kernels (forced at 5000, automatic at
    # 40000)
    z, y = _split_case(40, C, C + 1)
    ext.set_params(7 if C < 24576 else 0, 512)
    print(f"split drop-in ops C={C}", flush=True)
    zt, yt = to_dev(dev, z, y)
    ref = oracle.definition(z, y)
    H, losses, mean, kappa, sel = ext.fw_forward_small(zt, yt)
    grad = ext.fw_backward_small(yt, sel, kappa)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(sel.cpu().numpy(), z > ref["tau"][:, None])
    assert_parity(dict(H=H.cpu().numpy(), loss=losses.cpu().numpy(), mean=float(mean.cpu()),
                       kappa=kappa.cpu().numpy(), grad=grad.cpu().numpy()), ref, z)
    H, losses, mean, kappa, cbuf, cidx, ccnt = ext.fw_forward(zt, yt)
    grad = ext.fw_backward(zt, yt, H, kappa, cbuf, cidx, ccnt)
    torch.cuda.synchronize()
    cnt, cb, ci = ccnt.cpu().numpy(), cbuf.cpu().numpy(), cidx.cpu().numpy()
    np.testing.assert_array_equal(cnt, ref["kappa"])
    for r in range(z.shape[0]):
        idx = ci[r, :cnt[r]]
        assert np.array_equal(np.sort(idx), np.nonzero(z[r] > ref["tau"][r])[0]), f"row {r} support"
        assert bits_equal(cb[r, :cnt[r]], z[r, idx])
    assert_parity(dict(H=H.cpu().numpy(), loss=losses.cpu().numpy(), mean=float(mean.cpu()),
                       kappa=kappa.cpu().numpy(), grad=grad.cpu().numpy()), ref, z)


def test_split_rows_non_finite_like_block_rows(ext, dev, reset_params):
    # rows with +inf, NaN or no finite entry: the split kernels give what one block per row gives
    rng = np.random.default_rng(11)
    C = 20000
    z = rng.standard_normal((8, C)).astype(np.float32)
    z[0, 17000] = np.inf
    z[1, ::3] = np.nan
    z[2, 1024:2048] = -np.inf
    z[3] = -np.inf
    z[4] = np.nan
    z[5, :16384] = -np.inf
    z[6, 5] = np.inf
    z[6, 19999] = np.nan
    y = np.array([17000, 1, 1500, 3, 4, 19999, 5, 0])
    zt, yt = to_dev(dev, z, y)
    outs = []
    for path in (7, 2):
        ext.set_params(path, 512)
        print(f"non-finite rows path={path}", flush=True)
        outs.append(fused(ext, zt, yt))
    for k in ("H", "loss", "kappa", "grad"):
        a, b = outs[0][k], outs[1][k]
        assert (bits_equal(a, b) if a.dtype == np.float32 else np.array_equal(a, b)), k
    # finite rows against the oracle
    fin = [2, 5, 7]
    assert_parity({k: outs[0][k][fin] for k in ("H", "loss", "kappa", "grad")}, oracle.definition(z[fin], y[fin],
                  scale=1.0 / 8), z[fin])


# ---------------------------------------------------------------- shapes, layouts, special values

@pytest.mark.parametrize("C", [1, 2, 3, 5, 10, 37, 63, 64, 65, 255, 257, 999, 1001, 1023, 1025, 2049, 5000, 10001,
                               16384, 16385, 20000])
def test_shapes(ext, dev, C):
    rng = np.random.default_rng(C + 11)
    N = 67
    z = (rng.standard_normal((N, C)) * rng.choice([0.01, 1.0, 10.0], size=(N, 1))).astype(np.float32)
    y = rng.integers(0, C, N)
    print(f"shape N={N} C={C}", flush=True)
    assert_parity(fused(ext, *to_dev(dev, z, y)), oracle.definition(z, y), z)


@pytest.mark.parametrize("C", [4, 16, 17, 32, 33, 100, 128, 129, 256])
@pytest.mark.parametrize("N", [1, 2, 3, 5, 131])
def test_short_rows_groups(ext, dev, N, C):
    # short rows run R = 2 or 4 rows per wavefront iteration: every remainder of N by R, flat rows
    # (more candidates than lanes per row) and exact ties
    rng = np.random.default_rng(N * 1000 + C)
    z = rng.standard_normal((N, C)).astype(np.float32)
    z[::3] *= np.float32(0.01)
    z[1::4] = np.round(z[1::4] * 2) / 2
    y = rng.integers(0, C, N)
    print(f"short rows N={N} C={C}", flush=True)
    assert_parity(fused(ext, *to_dev(dev, z, y)), oracle.definition(z, y), z)
    zt, yt = to_dev(dev, z, y)
    H, losses, mean, kappa, sel = ext.fw_forward_small(zt, yt)
    torch.cuda.synchronize()
    ref = oracle.definition(z, y)
    np.testing.assert_array_equal(sel.cpu().numpy(), z > ref["tau"][:, None])


@pytest.mark.parametrize("K", [1, 2, 3, 7, 10, 100, 257, 1000, 4097, 40000])
def test_row_families(ext, dev, K):
    """Every row family (ties, constant, sorted, two-level, outlier, flat, heavy tails, -inf) at K
    from 1 to 40000: bit-exact against the oracle, and within the reference harness's tolerances
    against its fp64 sort recipe (CE_FW_perf.py:137-177)."""
    from test_oracle import fp64_sort_recipe
    z, y, _ = data.families(K, rows=4, seed=K + 1)
    print(f"families K={K} rows={z.shape[0]}", flush=True)
    ref = oracle.definition(z, y)
    out = fused(ext, *to_dev(dev, z, y))
    assert_parity(out, ref, z)
    H, kappa, grad, loss = fp64_sort_recipe(z, y, 1.0 / z.shape[0])
    ok = (ref["flags"] & 1) == 0
    np.testing.assert_array_equal(out["kappa"][ok], kappa[ok])
    np.testing.assert_allclose(out["H"], H, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out["loss"], loss, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out["grad"][ok], grad[ok], rtol=1e-5, atol=1e-6)


def test_edge_rows(ext, dev):
    z, y = data.edge_rows()
    print("edge rows", flush=True)
    ref = oracle.definition(z, y)
    out = fused(ext, *to_dev(dev, z, y))
    assert_parity(out, ref, z)
    # closed forms
    C = z.shape[1]
    assert out["kappa"][0] == C and out["kappa"][2] == 1
    assert out["loss"][2] == np.float32(0.0)                        # 1 - 5 + (5 - 1)


def test_label_at_minus_inf_and_bad_label(ext, dev):
    z = np.zeros((3, 8), np.float32)
    z[:, 5] = -np.inf
    y = np.array([5, 8, -1], np.int64)          # -inf label, then labels out of range
    out = fused(ext, *to_dev(dev, z, y))
    assert np.isposinf(out["loss"][0])
    assert np.isnan(out["loss"][1]) and np.isnan(out["loss"][2])
    assert np.all(out["kappa"] == 7)
    # out-of-range labels leave the gradient without the label term
    np.testing.assert_array_equal(out["grad"][1], np.where(z[1] > out["H"][1], np.float32((1 / 3) / 7), 0))


def test_misaligned_and_strided_inputs(ext, dev):
    rng = np.random.default_rng(5)
    big = torch.from_numpy(rng.standard_normal((40, 1001)).astype(np.float32)).to(dev)
    zt = big[:, 1:]                              # non-contiguous view, C = 1000
    yt = torch.from_numpy(rng.integers(0, 1000, 40)).to(dev)
    z = zt.cpu().numpy()
    ref = oracle.definition(z, yt.cpu().numpy())
    assert_parity(fused(ext, zt, yt), ref, z)
    flat = torch.from_numpy(rng.standard_normal(40 * 1000 + 1).astype(np.float32)).to(dev)
    zt2 = flat[1:].view(40, 1000)                # contiguous but only 4-byte aligned
    z2 = zt2.cpu().numpy()
    assert_parity(fused(ext, zt2, yt), oracle.definition(z2, yt.cpu().numpy()), z2)


@pytest.mark.parametrize("N,C,off", [(300, 1000, 0), (300, 996, 4), (5, 996, 4), (300, 1000, 4), (300, 480, 4),
                                      (300, 2000, 0), (300, 1996, 12), (300, 64, 4), (300, 500, 8), (300, 1020, 0),
                                      (300, 252, 0)])
def test_line_aligned_windows(ext, dev, reset_params, N, C, off):
    """Register rows read and written through line-aligned windows (path 1) against the oracle and
    bit-for-bit against path 8 (no windows), with logits and gradient both starting `off` floats
    into a 128-byte line; labels include both row ends; the floats around the gradient rows stay
    untouched.  (996, 4) and (1996, 12) take every shift 0..7; in (1000, 4), (500, 8), (1020, 0)
    and (252, 0) only the rows whose window fits the tier take one, the others plain addressing."""
    rng = np.random.default_rng(N + C + off)
    pad = 64
    zbuf = torch.from_numpy(rng.standard_normal(N * C + pad).astype(np.float32)).to(dev)
    zt = zbuf[off:off + N * C].view(N, C)
    y = rng.integers(0, C, N)
    y[:4] = [0, C - 1, C - 1, 0][:min(4, N)]
    yt = torch.from_numpy(y).to(dev)
    z = zt.cpu().numpy()
    ref = oracle.definition(z, y)
    outs = []
    for path in (1, 8):
        ext.set_params(path, 512)
        gbuf = torch.full((N * C + pad,), 7.0, device=dev)
        out = fwloss_capi.forward_backward(zt, yt, grad=gbuf[off:off + N * C].view(N, C))
        torch.cuda.synchronize()
        g = gbuf.cpu().numpy()
        assert np.all(g[:off] == 7.0) and np.all(g[off + N * C:] == 7.0)
        res = {k: v.cpu().numpy() for k, v in out.items()}
        np.testing.assert_array_equal(res["kappa"], ref["kappa"])
        assert bits_equal(res["H"], ref["H"]) and bits_equal(res["loss"], ref["loss"])
        assert bits_equal(res["grad"], ref["grad"])
        outs.append(res)
    for k in ("H", "loss", "kappa", "grad", "mean"):
        assert bits_equal(outs[0][k], outs[1][k]), k


@pytest.mark.parametrize("N,C,off", [(300, 1000, 0), (300, 996, 4), (300, 1020, 0), (300, 64, 4), (5, 1000, 0)])
def test_offset_mask_rows(ext, dev, reset_params, N, C, off):
    """The drop-in mask forward (fw_forward_small) on register rows (paths 1 and 8; mask rows keep
    plain addressing on both), logits starting `off` floats into a 128-byte line: the support mask,
    H, losses, kappa and the gradient from the mask against the oracle, and the two paths
    bit-for-bit."""
    rng = np.random.default_rng(N + 7 * C + off)
    zbuf = torch.from_numpy(rng.standard_normal(N * C + 64).astype(np.float32)).to(dev)
    zt = zbuf[off:off + N * C].view(N, C)
    y = rng.integers(0, C, N)
    y[:2] = [0, C - 1][:min(2, N)]
    yt = torch.from_numpy(y).to(dev)
    z = zt.cpu().numpy()
    ref = oracle.definition(z, y)
    outs = []
    for path in (1, 8):
        ext.set_params(path, 512)
        H, losses, mean, kappa, sel = ext.fw_forward_small(zt, yt)
        grad = ext.fw_backward_small(yt, sel, kappa)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(sel.cpu().numpy(), z > ref["tau"][:, None])
        out = dict(H=H.cpu().numpy(), loss=losses.cpu().numpy(), mean=float(mean.cpu()), kappa=kappa.cpu().numpy(),
                   grad=grad.cpu().numpy())
        assert_parity(out, ref, z)
        outs.append(out)
    for k in ("H", "loss", "kappa", "grad"):
        assert bits_equal(outs[0][k], outs[1][k]), k


def test_empty_batch(ext, dev):
    zt = torch.empty((0, 10), device=dev)
    yt = torch.empty((0,), dtype=torch.int64, device=dev)
    H, loss, mean, kappa, grad = ext.fw_forward_backward(zt, yt)
    assert H.shape == (0,) and grad.shape == (0, 10) and torch.isnan(mean).item()
    H, loss, mean, kappa, sel = ext.fw_forward_small(zt, yt)
    assert sel.shape == (0, 10)


def test_deterministic(ext, dev):
    z, y = data.make("cfg4", N=64, seed=9)
    zt, yt = to_dev(dev, z, y)
    a = fused(ext, zt, yt)
    b = fused(ext, zt, yt)
    for k in ("H", "loss", "kappa", "grad"):
        assert bits_equal(a[k], b[k]) if a[k].dtype == np.float32 else np.array_equal(a[k], b[k])
    assert a["mean"] == b["mean"]


@pytest.mark.parametrize("N,C", [(1 << 20, 16), (300000, 100), (1500, 1000), (700, 3000)])
def test_mean_over_many_blocks(ext, dev, N, C):
    """The mean of grids from a few hundred blocks to several thousand (several batches of partial
    loads in the one-block finishing kernel): equal to the fp64 mean of the per-row losses, and
    bit-identical on a repeated call (fixed summation order)."""
    rng = np.random.default_rng(N + C)
    z = rng.standard_normal((N, C), dtype=np.float32)
    y = rng.integers(0, C, N, dtype=np.int64)
    zt, yt = to_dev(dev, z, y)
    out = []
    for rdiv in (float(N), 1.0, float(N)):
        H, loss, mean, kappa, grad = ext.fw_forward_backward(zt, yt, 1.0 / N, rdiv)
        torch.cuda.synchronize()
        ref = loss.double().sum().item() / rdiv
        assert abs(mean.item() - ref) <= 1e-6 * max(1.0, abs(ref)), (rdiv, mean.item(), ref)
        out.append(mean.item())
    assert out[0] == out[2]


# ---------------------------------------------------------------- full-size configurations

def _row_properties(zt, yt, H, loss, kappa, grad, scale):
    """Size-independent checks on the device in fp64: the support is {z > H}, the threshold solves
    sum(z - tau)_+ = 1, and the gradient is the closed form."""
    z64 = zt.double()
    sel = zt > H[:, None]
    k = sel.sum(1)
    assert torch.equal(k.int(), kappa), "kappa != |{z > H}|"
    S = torch.where(sel, z64, torch.zeros_like(z64)).sum(1)
    tau = (S - 1.0) / k.double()
    # H is the largest float <= tau
    assert torch.all(H.double() <= tau) and torch.all(torch.nextafter(H, torch.full_like(H, np.inf)).double() > tau)
    # sum over the support of (z - tau) = 1, and nothing outside the support is above tau
    resid = torch.where(sel, z64 - tau[:, None], torch.zeros_like(z64)).sum(1) - 1.0
    assert resid.abs().max().item() < 1e-9
    assert torch.all(torch.where(sel, torch.full_like(z64, -np.inf), z64).max(1).values <= tau)
    zy = z64.gather(1, yt[:, None])[:, 0]
    assert torch.allclose(loss.double(), (1.0 - zy) + tau, rtol=1e-6, atol=1e-6)
    inv = (scale / k.double()).float()
    expect = torch.where(sel, inv[:, None], torch.zeros_like(zt))
    expect.scatter_(1, yt[:, None], expect.gather(1, yt[:, None]) - np.float32(scale))
    assert torch.equal(grad, expect), "grad differs from the closed form"
    assert grad.double().sum(1).abs().max().item() < 1e-6


@pytest.mark.parametrize("cfg", ["cfg2", "cfg3", "cfg4", "cfg5"])
def test_full_size(ext, dev, cfg):
    z, y = data.make(cfg, seed=0)
    N = z.shape[0]
    print(f"full size {cfg} N={N} C={z.shape[1]}", flush=True)
    zt, yt = to_dev(dev, z, y)
    H, loss, mean, kappa, grad = ext.fw_forward_backward(zt, yt)
    torch.cuda.synchronize()
    _row_properties(zt, yt, H, loss, kappa, grad, 1.0 / N)
    assert abs(mean.item() - loss.double().mean().item()) <= 1e-6 * max(1.0, abs(mean.item()))
    rows = np.random.default_rng(0).choice(N, size=min(N, 64), replace=False)
    ref = oracle.definition(z[rows], y[rows], scale=1.0 / N)
    sub = dict(H=H[rows].cpu().numpy(), loss=loss[rows].cpu().numpy(), kappa=kappa[rows].cpu().numpy(),
               grad=grad[rows].cpu().numpy(), mean=None)
    assert_parity(sub, ref, z[rows])
    del zt, grad
    torch.cuda.empty_cache()


@pytest.mark.parametrize("N,C", [(1_000_003, 16), (300_001, 100), (65_537, 1025), (9_999, 8193), (6_200, 8192),
                                 (4_201, 12_000), (4_095, 8192)])
def test_large_batches(ext, dev, N, C):
    # grid limits of every kernel family: more than 2048 blocks of short rows, odd N, unaligned C;
    # fp32 rows of 8192-32000 elements in batches of >= 32M elements run in two passes (6200 x
    # 8192; 4095 x 8192 stays just below that and runs in one)
    rng = np.random.default_rng(N + C)
    z = rng.standard_normal((N, C), dtype=np.float32)
    y = rng.integers(0, C, N)
    print(f"large batch N={N} C={C}", flush=True)
    zt, yt = to_dev(dev, z, y)
    H, loss, mean, kappa, grad = ext.fw_forward_backward(zt, yt)
    torch.cuda.synchronize()
    _row_properties(zt, yt, H, loss, kappa, grad, 1.0 / N)
    assert abs(mean.item() - loss.double().mean().item()) <= 1e-6 * max(1.0, abs(mean.item()))
    rows = rng.choice(N, size=48, replace=False)
    ref = oracle.definition(z[rows], y[rows], scale=1.0 / N)
    sub = dict(H=H[rows].cpu().numpy(), loss=loss[rows].cpu().numpy(), kappa=kappa[rows].cpu().numpy(),
               grad=grad[rows].cpu().numpy(), mean=None)
    assert_parity(sub, ref, z[rows])
    del zt, grad
    torch.cuda.empty_cache()


# ---------------------------------------------------------------- graphs and streams

@pytest.mark.parametrize("cfg,N", [("cfg2", 1000), ("cfg3", 1000), ("cfg4", 512), ("cfg5", 16)])
def test_graph_capture_replays(ext, dev, cfg, N):
    """The fused op allocates nothing on the device path and keeps no state in its workspace, so it
    can be captured in a HIP graph: every replay must equal the eager result.  The shapes take the register, segmented, two-pass
    (read, fill, scatter) and split-row paths."""
    z, y = data.make(cfg, N=N, seed=21)
    zt, yt = to_dev(dev, z, y)
    eager = ext.fw_forward_backward(zt, yt)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):   # warm the per-stream workspace outside the capture
            ext.fw_forward_backward(zt, yt)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ext.fw_forward_backward(zt, yt)
    print(f"graph replays {cfg} N={N}", flush=True)
    for it in range(5):
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(out, eager):
            assert torch.equal(a, b), f"replay {it} differs from the eager result"
        _ = ext.fw_forward_backward(zt, yt)   # eager work between replays
        torch.cuda.synchronize()


def test_concurrent_streams(ext, dev):
    """Two streams run the fused op concurrently, each with its own cached workspace."""
    z1, y1 = data.make("cfg2", N=4096, seed=31)
    z2, y2 = data.make("cfg3", N=8192, seed=32)
    a1, b1 = to_dev(dev, z1, y1)
    a2, b2 = to_dev(dev, z2, y2)
    r1 = ext.fw_forward_backward(a1, b1)
    r2 = ext.fw_forward_backward(a2, b2)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    print("concurrent streams", flush=True)
    for _ in range(10):
        with torch.cuda.stream(s1):
            o1 = ext.fw_forward_backward(a1, b1)
        with torch.cuda.stream(s2):
            o2 = ext.fw_forward_backward(a2, b2)
        outs.append((o1, o2))
    torch.cuda.synchronize()
    for o1, o2 in outs:
        for a, b in zip(o1, r1):
            assert torch.equal(a, b)
        for a, b in zip(o2, r2):
            assert torch.equal(a, b)


# ---------------------------------------------------------------- autograd API and the C ABI

@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_autograd(ext, dev, reduction):
    z, y = data.make("cfg2", N=300, seed=4)
    zt, yt = to_dev(dev, z, y)
    zt.requires_grad_(True)
    loss = ext.familywise_loss(zt, yt, reduction)
    N = z.shape[0]
    ref = oracle.definition(z, y, scale=1.0 / N if reduction == "mean" else 1.0)
    if reduction == "none":
        go = torch.linspace(0.5, 2.0, N, device=dev)
        go[::3] = 1.0
        loss.backward(go)
        expect = ref["grad"] * go.cpu().numpy()[:, None]
        np.testing.assert_array_equal(loss.detach().cpu().numpy(), ref["loss"])
    else:
        (loss * 3.0).backward()
        expect = ref["grad"] * np.float32(3.0)
        tot = ref["loss"].astype(np.float64).sum() / (N if reduction == "mean" else 1)
        assert abs(loss.item() - tot) <= 1e-6 * max(1.0, abs(tot))
    assert bits_equal(zt.grad.cpu().numpy(), expect.astype(np.float32))


def test_fw_loss_grad_api(ext, dev):
    """fwloss.fw_loss_grad: the outputs and dtypes of the reference's fwcpp.fw_loss_grad."""
    z, y = data.make("cfg3", N=200, seed=8)
    zt, yt = to_dev(dev, z, y)
    L, G, k = ext.fw_loss_grad(zt, yt, 0.25, 2 ** 62, 100000, True)
    assert L.dtype == torch.float64 and G.dtype == torch.float32 and k.dtype == torch.int64
    ref = oracle.definition(z, y, scale=0.25)
    np.testing.assert_array_equal(k.cpu().numpy(), ref["kappa"])
    # the fp64 losses (1 - z_y) + tau: the oracle's own fp64 values, bit for bit
    np.testing.assert_array_equal(L.cpu().numpy(), ref["loss64"])
    assert bits_equal(G.cpu().numpy(), ref["grad"])


def test_c_abi_direct(ext, dev):
    z, y = data.make("cfg2", N=256, seed=6)
    zt, yt = to_dev(dev, z, y)
    out = fwloss_capi.forward_backward(zt, yt)
    torch.cuda.synchronize()
    got = {k: (v.cpu().numpy() if v.dim() else float(v.cpu())) for k, v in out.items()}
    assert_parity(got, oracle.definition(z, y), z)


@pytest.mark.parametrize("C", [32000, 40000])
def test_long_rows_one_pass_without_workspace(ext, dev, C):
    # >= 384 rows of >= 32000 elements run in two passes when the workspace has room; without a
    # workspace (no mean requested) the one-pass block kernel runs: both against the oracle
    import ctypes
    rng = np.random.default_rng(C)
    N = 520
    z = rng.standard_normal((N, C)).astype(np.float32)
    z[::7] *= np.float32(0.01)
    y = rng.integers(0, C, N)
    zt, yt = to_dev(dev, z, y)
    ref = oracle.definition(z, y)
    L = fwloss_capi.lib()
    H = torch.empty(N, device=dev)
    loss = torch.empty(N, device=dev)
    kappa = torch.empty(N, dtype=torch.int32, device=dev)
    grad = torch.empty_like(zt)
    P = ctypes.c_void_p
    print(f"one pass without workspace C={C}", flush=True)
    rc = L.fwl_forward_backward(P(zt.data_ptr()), P(yt.data_ptr()), N, C, 1.0 / N, float(N), P(H.data_ptr()),
                                P(loss.data_ptr()), None, P(kappa.data_ptr()), P(grad.data_ptr()), None, 0,
                                P(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    assert_parity(dict(H=H.cpu().numpy(), loss=loss.cpu().numpy(), kappa=kappa.cpu().numpy(),
                       grad=grad.cpu().numpy()), ref, z)
    print(f"two passes C={C}", flush=True)
    assert_parity(fused(ext, zt, yt), ref, z)
