"""Pins the CPU oracle (oracle/fwl_oracle.c) before it is trusted as the checker of the HIP path.

* exact rational brute force: tau = max over ALL non-empty subsets S of (sum(S) - 1)/|S| (a
  different formula from the sorted-prefix one the oracle uses), kappa = |{z > tau}|;
* the defining root: sum_j max(z_j - tau, 0) = 1;
* closed forms: C = 1, constant rows, a top gap >= 1, two-level rows;
* invariants: shift equivariance, permutation invariance, gradient rows summing to zero;
* the golden vectors written by the reference's own CPU path (tests/golden/, make_golden.py);
* the compiled reference itself (oracle/_ref) on fresh seeded inputs, when it is built;
* the streaming restatement of src/cpu against the definition.
"""
import glob
import itertools
import os
from fractions import Fraction

import numpy as np
import pytest

import fwloss_data as data
import oracle

HERE = os.path.dirname(os.path.abspath(__file__))


def exact_tau(row):
    """max over all non-empty subsets of (sum - 1)/size, in exact rational arithmetic."""
    v = [Fraction(float(x)) for x in row if np.isfinite(x)]
    best = None
    for k in range(1, len(v) + 1):
        for comb in itertools.combinations(v, k):
            h = (sum(comb) - 1) / k
            if best is None or h > best:
                best = h
    return best


def largest_float_le(q):
    f = np.float32(float(q))
    if Fraction(float(f)) > q:
        f = np.nextafter(f, np.float32(-np.inf))
    return f


def random_small_rows(rng, count):
    rows = []
    for _ in range(count):
        C = int(rng.integers(1, 10))
        kind = rng.integers(0, 4)
        if kind == 0:
            r = rng.standard_normal(C)
        elif kind == 1:
            r = rng.integers(-4, 5, C) * 0.25            # dyadic, exact ties
        elif kind == 2:
            r = rng.standard_normal(C) * 0.05            # flat: long supports
        else:
            r = np.repeat(rng.standard_normal(max(1, C // 2)), 2)[:C]   # pairs of ties
        rows.append(np.asarray(r, dtype=np.float32))
    return rows


def test_definition_matches_exact_subset_brute_force():
    rng = np.random.default_rng(2024)
    for row in random_small_rows(rng, 300):
        C = row.size
        y = np.array([rng.integers(0, C)])
        out = oracle.definition(row[None, :], y, scale=0.5)
        tau = exact_tau(row)
        kappa = sum(Fraction(float(x)) > tau for x in row)
        assert out["kappa"][0] == kappa, (row, tau)
        assert out["H"][0] == largest_float_le(tau), (row, tau)
        assert abs(out["tau"][0] - float(tau)) <= 1e-12 * max(1.0, abs(float(tau)))
        assert out["flags"][0] == 0
        inv = np.float32(0.5 / kappa)
        g = np.where(np.array([Fraction(float(x)) > tau for x in row]), inv, np.float32(0)).astype(np.float32)
        g[y[0]] -= np.float32(0.5)
        np.testing.assert_array_equal(out["grad"][0], g)
        # the defining root: sum of the positive parts above tau is exactly 1
        assert sum(max(Fraction(float(x)) - tau, Fraction(0)) for x in row) == 1


def test_closed_forms():
    C = 12
    # C = 1: kappa = 1, tau = z - 1, loss 0, gradient 0
    out = oracle.definition(np.array([[3.5]], np.float32), np.array([0]), scale=1.0)
    assert out["kappa"][0] == 1 and out["loss"][0] == 0 and out["grad"][0, 0] == 0
    # constant row v: kappa = C, tau = v - 1/C, loss = 1 - 1/C
    out = oracle.definition(np.full((1, C), 2.0, np.float32), np.array([3]), scale=1.0)
    assert out["kappa"][0] == C
    assert abs(out["tau"][0] - (2.0 - 1.0 / C)) < 1e-15 and abs(out["loss64"][0] - (1 - 1.0 / C)) < 1e-15
    # top gap >= 1: kappa = 1, tau = max - 1, loss = max - z_y
    z = np.array([[1.0, 3.0, 2.0, -1.0]], np.float32)
    out = oracle.definition(z, np.array([2]), scale=1.0)
    assert out["kappa"][0] == 1 and out["tau"][0] == 2.0 and out["loss64"][0] == 1.0
    # two levels: p copies of a and q of b, a - b = 0.5: with p = 4, tau_p = a - 1/4 > b -> kappa 4
    z = np.array([[2.0] * 4 + [1.5] * 6], np.float32)
    out = oracle.definition(z, np.array([0]), scale=1.0)
    assert out["kappa"][0] == 4 and out["tau"][0] == 1.75
    # with p = 1 the whole row: tau = (2 + 6*1.5 - 1)/7 = 10/7 < 1.5 -> kappa 7
    z = np.array([[2.0] + [1.5] * 6], np.float32)
    out = oracle.definition(z, np.array([0]), scale=1.0)
    assert out["kappa"][0] == 7 and abs(out["tau"][0] - 10.0 / 7.0) < 1e-15
    # exact tie at the boundary: [4, 4, 3.5, 3.5, ...]: tau = 3.5 exactly, strict support = 2
    z = np.array([[4.0, 4.0, 3.5, 3.5, -1.0, -1.0]], np.float32)
    out = oracle.definition(z, np.array([0]), scale=1.0)
    assert out["kappa"][0] == 2 and out["tau"][0] == 3.5 and out["H"][0] == 3.5


def test_invariants():
    rng = np.random.default_rng(7)
    # multiples of 2^-10 within +-8: the shifts below are exact in fp32
    z = (np.round(rng.standard_normal((200, 37)) * 1024) / 1024).astype(np.float32)
    y = rng.integers(0, 37, 200)
    base = oracle.definition(z, y, scale=1.0)
    # shift by a few units: tau shifts, kappa and loss do not
    for c in (1.0, -2.0, 8.0):
        sh = oracle.definition(z + np.float32(c), y, scale=1.0)
        np.testing.assert_array_equal(sh["kappa"], base["kappa"])
        np.testing.assert_allclose(sh["tau"], base["tau"] + c, rtol=0, atol=1e-12)
        np.testing.assert_allclose(sh["loss64"], base["loss64"], rtol=0, atol=1e-12)
    # permutation of the classes (with the label)
    perm = rng.permutation(37)
    inv = np.argsort(perm)
    pm = oracle.definition(z[:, perm], inv[y], scale=1.0)
    np.testing.assert_array_equal(pm["kappa"], base["kappa"])
    np.testing.assert_array_equal(pm["H"], base["H"])
    np.testing.assert_array_equal(pm["grad"][:, inv], base["grad"])
    # gradient rows sum to kappa * inv - 1 ~ 0
    assert np.abs(base["grad"].astype(np.float64).sum(1)).max() < 1e-6


def test_single_pass_restatement_matches_definition():
    rng = np.random.default_rng(3)
    for C in (7, 100, 1000, 5000):
        z = (rng.standard_normal((64, C)) * rng.choice([0.001, 0.1, 1.0, 10.0], size=(64, 1))).astype(np.float32)
        z[::9] = np.round(z[::9] * 4) / 4
        y = rng.integers(0, C, 64)
        d = oracle.definition(z, y)
        s = oracle.single_pass(z, y)
        np.testing.assert_array_equal(s["kappa"], d["kappa"])
        np.testing.assert_allclose(s["loss64"], d["loss64"], rtol=1e-12, atol=1e-12)
        np.testing.assert_array_equal(s["grad"], d["grad"])
    # work cap 0 forces the fallback on every row that needs more than one Newton step
    s0 = oracle.single_pass(z, y, cap_factor=0)
    np.testing.assert_array_equal(s0["kappa"], d["kappa"])


F32_GOLDEN = sorted(p for p in glob.glob(os.path.join(HERE, "golden", "golden_*.npz")) if not p.endswith("_f64.npz"))


@pytest.mark.parametrize("path", F32_GOLDEN, ids=lambda p: os.path.basename(p))
def test_oracle_reproduces_reference_golden_vectors(path):
    g = np.load(path)
    z, y, scale = g["z"], g["y"], float(g["scale"])
    out = oracle.definition(z, y, scale=scale)
    np.testing.assert_array_equal(out["kappa"], g["kappa"])
    # rows with |z| >= 2^53 are outside fp64's exact regime (max - 1 is not representable): both
    # sides round tau differently there, so their losses agree to 1e-9 only
    big = np.abs(z).max(1) >= 2.0 ** 53
    np.testing.assert_allclose(out["loss64"][~big], g["L"][~big], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out["loss64"][big], g["L"][big], rtol=1e-9)
    G = np.zeros_like(z)
    G[g["g_rows"], g["g_cols"]] = g["g_vals"]
    np.testing.assert_array_equal(out["grad"], G)


def test_golden_fixtures_cover_every_configuration():
    names = {os.path.basename(p) for p in glob.glob(os.path.join(HERE, "golden", "golden_*.npz"))}
    assert {f"golden_cfg{i}.npz" for i in range(1, 6)} | {"golden_edges.npz"} <= names


def test_oracle_matches_compiled_reference():
    ref = oracle.load_ref()
    if ref is None:
        pytest.skip("oracle/_ref not built here (the reference sources are needed to build it)")
    import torch
    for cfg, N in (("cfg1", 1024), ("cfg2", 256), ("cfg3", 2048), ("cfg4", 8), ("cfg5", 4)):
        z, y = data.make(cfg, N=N, seed=99)
        L, G, k = ref.fw_loss_grad(torch.from_numpy(z), torch.from_numpy(y), 1.0 / N, 2 ** 62, 100000, True)
        out = oracle.definition(z, y)
        np.testing.assert_array_equal(out["kappa"], k.numpy())
        np.testing.assert_allclose(out["loss64"], L.numpy(), rtol=1e-12, atol=1e-12)
        np.testing.assert_array_equal(out["grad"], G.numpy())


F64_CASES = ("gauss", "ties", "wide", "flat")


@pytest.mark.parametrize("name", F64_CASES)
def test_f64_oracle_reproduces_reference_golden_vectors(name):
    """float64 logits: the numpy definition against the compiled reference's run_generic<double>
    (fw_cpu.cpp:697-703): kappa and the gradient bit-identical, losses within 1e-15 relative (the
    reference writes the loss as 1 + (thr - z_y) + (tau - thr), fw_cpu.cpp:614)."""
    g = np.load(os.path.join(HERE, "golden", "golden_f64.npz"))
    z, y, scale = g[f"{name}_z"], g[f"{name}_y"], float(g[f"{name}_scale"])
    out = oracle.definition_f64(z, y, scale)
    np.testing.assert_array_equal(out["kappa"], g[f"{name}_kappa"])
    np.testing.assert_allclose(out["loss"], g[f"{name}_L"], rtol=1e-15, atol=1e-15)
    G = np.zeros_like(z)
    G[g[f"{name}_g_rows"], g[f"{name}_g_cols"]] = g[f"{name}_g_vals"]
    np.testing.assert_array_equal(out["grad"], G)


def test_f64_oracle_matches_exact_subset_brute_force():
    """tau of the fp64 definition is within an ulp of the exact rational max over all subsets, kappa
    is the exact support size and the loss is the fp64 formula (small rows, ties included)."""
    rng = np.random.default_rng(64)
    for row in random_small_rows(rng, 300):
        row = row.astype(np.float64)
        if rng.integers(0, 2):
            row = row + rng.standard_normal(row.size) * 1e-9     # values that are not fp32
        out = oracle.definition_f64(row[None, :], np.zeros(1, np.int64), 1.0)
        tau = exact_tau(row)
        t = out["tau"][0]
        # fp64 prefix sums round once per term: a few ulps of the magnitudes involved
        scale_ = Fraction(float(np.abs(row).max())) + abs(tau) + 1
        assert abs(Fraction(float(t)) - tau) <= scale_ * row.size * Fraction(1, 2 ** 52)
        assert out["kappa"][0] == sum(Fraction(float(x)) > tau for x in row)
        assert out["loss"][0] == (1.0 - row[0]) + t


def test_f64_oracle_matches_compiled_reference():
    ref = oracle.load_ref()
    if ref is None:
        pytest.skip("oracle/_ref not built here (the reference sources are needed to build it)")
    import torch
    rng = np.random.default_rng(5)
    for N, C in ((64, 1000), (16, 7), (8, 20000)):
        z = rng.standard_normal((N, C)) * rng.uniform(0.1, 5.0)
        y = rng.integers(0, C, N).astype(np.int64)
        L, G, k = ref.fw_loss_grad(torch.from_numpy(z), torch.from_numpy(y), 1.0 / N, 2 ** 62, 100000, True)
        out = oracle.definition_f64(z, y)
        np.testing.assert_array_equal(out["kappa"], k.numpy())
        np.testing.assert_allclose(out["loss"], L.numpy(), rtol=1e-15, atol=1e-15)
        np.testing.assert_array_equal(out["grad"], G.numpy())


def fp64_sort_recipe(z, y, scale):
    """The reference GPU harness's check recipe (benchmarks/cuda_benchmarks/CE_FW_perf.py:137-168),
    restated with torch fp64 CPU ops: sort descending, prefix sums, H_k = (S_k - 1)/k, H = max_k,
    kappa = first argmax + 1, grad = [z > H]/kappa - [j = y], times scale."""
    import torch
    z64 = torch.from_numpy(z).double()
    srt = torch.sort(z64, dim=1, descending=True).values
    S = srt.cumsum(dim=1)
    k = torch.arange(1, z.shape[1] + 1, dtype=torch.float64)
    H, idx = ((S - 1.0) / k).max(dim=1)
    kappa = idx + 1
    grad = (z64 > H[:, None]).double() / kappa[:, None].double()
    grad[torch.arange(z.shape[0]), torch.from_numpy(y)] -= 1.0
    loss = 1.0 - z64[torch.arange(z.shape[0]), torch.from_numpy(y)] + H
    return H.numpy(), kappa.numpy(), (grad * scale).numpy(), loss.numpy()


@pytest.mark.parametrize("K", [1, 2, 3, 7, 10, 100, 1000, 40000])
def test_oracle_matches_fp64_sort_recipe(K):
    """The oracle against the reference harness's own fp64 recipe on every row family, with the
    harness's tolerances (CE_FW_perf.py:170-177: kappa equal, the rest rtol 1e-5 / atol 1e-6).
    Rows where the fp64 argmax and the strict support count part ways (flag bit 1; only possible
    through fp64 rounding at an exact tie) are excluded from the kappa comparison."""
    z, y, _ = data.families(K, rows=3, seed=K)
    scale = 1.0 / z.shape[0]
    out = oracle.definition(z, y, scale=scale)
    H, kappa, grad, loss = fp64_sort_recipe(z, y, scale)
    ok = (out["flags"] & 1) == 0
    np.testing.assert_array_equal(out["kappa"][ok], kappa[ok])
    np.testing.assert_allclose(out["H"], H, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out["loss64"], loss, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out["grad"][ok], grad[ok], rtol=1e-5, atol=1e-6)
