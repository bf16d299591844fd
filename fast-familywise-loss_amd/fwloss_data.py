"""Seeded synthetic inputs for the benchmark configurations.

One generator per configuration, as the configurations are specified for this operator (logits and
int64 labels uniform in [0, C)); the reference seeds its GPU harness with torch.manual_seed(0)
(benchmarks/cuda_benchmarks/CE_FW_perf.py:91-92) and its CPU harness with default_rng(0)
(benchmarks/cpu_benchmarks/bench_cpu_e2e.py:30).  Inputs are produced on the host with numpy's
PCG64 so that the CPU checkers and the GPU see identical bytes.

    cfg1  N=1024,  C=10      N(0,1)
    cfg2  N=65536, C=1000    N(0,1)                                  (headline)
    cfg3  N=16384, C=100     0.5 * integers in [-8, 8]               (heavy exact ties)
    cfg4  N=8192,  C=32000   N(0,1), +4 on the label in 70% of rows
    cfg5  N=2048,  C=131072  Gumbel(0,1); 1% -inf, 0.1% +-0.0, labels kept finite
"""
import numpy as np

CONFIGS = {
    "cfg1": dict(N=1024, C=10),
    "cfg2": dict(N=65536, C=1000),
    "cfg3": dict(N=16384, C=100),
    "cfg4": dict(N=8192, C=32000),
    "cfg5": dict(N=2048, C=131072),
}


def make(cfg, N=None, seed=0):
    """(z float32 [N, C], y int64 [N]) for configuration ``cfg`` (N defaults to the config's)."""
    spec = CONFIGS[cfg]
    N = spec["N"] if N is None else N
    C = spec["C"]
    rng = np.random.default_rng(seed)
    y = rng.integers(0, C, size=N, dtype=np.int64)
    if cfg in ("cfg1", "cfg2"):
        z = rng.standard_normal((N, C), dtype=np.float32)
    elif cfg == "cfg3":
        z = (0.5 * rng.integers(-8, 9, size=(N, C))).astype(np.float32)
    elif cfg == "cfg4":
        z = rng.standard_normal((N, C), dtype=np.float32)
        boost = rng.random(N) < 0.7
        z[np.arange(N)[boost], y[boost]] += np.float32(4.0)
    elif cfg == "cfg5":
        u = rng.random((N, C), dtype=np.float32)
        u = np.clip(u, np.float32(1e-7), np.float32(1.0 - 6e-8))
        z = -np.log(-np.log(u))
        w = rng.random((N, C), dtype=np.float32)
        zy = z[np.arange(N), y].copy()
        z[w < 0.01] = -np.inf
        z[(w >= 0.01) & (w < 0.0105)] = 0.0
        z[(w >= 0.0105) & (w < 0.011)] = -0.0
        z[np.arange(N), y] = zy
        z = z.astype(np.float32, copy=False)
    else:
        raise KeyError(cfg)
    return np.ascontiguousarray(z, dtype=np.float32), y


DISTS = ("gauss", "laplace", "mixture")


def make_dist(dist, N, C, sigma=1.0, seed=0):
    """(z float32 [N, C], y int64 [N]) from the input distributions of the reference's GPU harness
    (benchmarks/cuda_benchmarks/data_io.py:8-83), swept there over sigma in {0.001, 0.01, 0.1, 1,
    10, 100} (CE_FW_perf.py:94-96):

        gauss    sigma * N(0, 1)                                  (data_io.py:8-21)
        laplace  Laplace(0, sigma / sqrt(2)), variance sigma^2    (data_io.py:23-42)
        mixture  each entry N(0, 1) or N(0, sigma^2), with probability 1/2 each (data_io.py:44-83)

    Labels are uniform in [0, C).  Drawn with numpy's PCG64 (float32 draws), so the CPU checkers
    and the GPU see identical bytes; the distributions are the reference's, the streams are not
    torch's."""
    if dist not in DISTS:
        raise KeyError(dist)
    rng = np.random.default_rng(seed)
    y = rng.integers(0, C, size=N, dtype=np.int64)
    s = np.float32(sigma)
    if dist == "gauss":
        z = rng.standard_normal((N, C), dtype=np.float32)
        z *= s
    elif dist == "laplace":
        # the difference of two standard exponentials is Laplace(0, 1)
        z = rng.standard_exponential((N, C), dtype=np.float32)
        z -= rng.standard_exponential((N, C), dtype=np.float32)
        z *= np.float32(sigma / np.sqrt(2.0))
    else:
        first = rng.random((N, C), dtype=np.float32) < np.float32(0.5)
        z = rng.standard_normal((N, C), dtype=np.float32)
        z[~first] *= s
    return np.ascontiguousarray(z, dtype=np.float32), y


FAMILIES = ("gauss", "ties", "constant", "sorted", "two_level", "outlier", "flat", "heavy", "neginf")


def families(K, rows=4, seed=0):
    """Rows of every family for row length K: (z float32 [len(FAMILIES) * rows, K], y int64, names).

    The families are those the reference's CPU test description names (ties, constant, sorted,
    two-level, outlier; src/cpu/README.md:87), plus flat rows (long supports), heavy tails and
    rows with -inf entries.
    """
    rng = np.random.default_rng(seed)
    out, names = [], []
    for fam in FAMILIES:
        for _ in range(rows):
            if fam == "gauss":
                r = rng.standard_normal(K)
            elif fam == "ties":
                r = 0.5 * rng.integers(-3, 4, K)
            elif fam == "constant":
                r = np.full(K, rng.standard_normal())
            elif fam == "sorted":
                r = np.sort(rng.standard_normal(K))
            elif fam == "two_level":
                a, gap = rng.standard_normal(), rng.uniform(0.0, 2.0)
                p = int(rng.integers(1, K + 1))
                r = np.r_[np.full(p, a), np.full(K - p, a - gap)]
                rng.shuffle(r)
            elif fam == "outlier":
                r = rng.standard_normal(K)
                r[rng.integers(0, K)] += 10.0
            elif fam == "flat":
                r = 1e-3 * rng.standard_normal(K)
            elif fam == "heavy":
                r = np.clip(rng.standard_cauchy(K), -1e6, 1e6)
            else:
                r = rng.standard_normal(K)
                r[rng.random(K) < 0.3] = -np.inf
                r[rng.integers(0, K)] = rng.standard_normal()
            out.append(r)
            names.append(fam)
    z = np.ascontiguousarray(np.stack(out).astype(np.float32))
    y = rng.integers(0, K, size=z.shape[0], dtype=np.int64)
    # keep labels off -inf entries, so every loss is finite
    for i in range(z.shape[0]):
        if not np.isfinite(z[i, y[i]]):
            y[i] = int(np.flatnonzero(np.isfinite(z[i]))[0])
    return z, y, names


def edge_rows():
    """Hand-made rows exercising the special cases of the definition: (z [R, C], y [R]) per C."""
    C = 16
    rows = [
        np.zeros(C),                                            # constant row: kappa = C
        np.full(C, 3.25),                                       # constant, shifted
        np.r_[5.0, np.zeros(C - 1)],                            # top gap >= 1: kappa = 1
        np.r_[1.0, 1.0, np.zeros(C - 2)],                       # gap exactly 1 below a tie pair
        np.r_[np.full(4, 2.0), np.full(C - 4, 1.0)],            # two levels
        np.r_[4.0, 4.0, 3.5, 3.5, np.full(C - 4, -1.0)],        # exact tie at the boundary
        np.r_[-0.0, 0.0, -0.0, 0.0, np.full(C - 4, -3.0)],      # signed zeros are equal
        np.r_[np.full(C - 1, -np.inf), 0.5],                    # -inf entries never selected
        np.linspace(-1.0, 1.0, C),                              # evenly spaced
        np.r_[1e-30, -1e-30, 1e-38, np.zeros(C - 3)],            # tiny magnitudes
        np.r_[1e30, 1e30 - 2**80, np.full(C - 2, -1e30)],       # huge magnitudes
        np.r_[np.float32(1) + np.float32(2**-23), 2.0, np.full(C - 2, -5.0)],
    ]
    z = np.stack([np.asarray(r, dtype=np.float64) for r in rows]).astype(np.float32)
    y = np.array([3, 0, 0, 1, 7, 2, 1, 15, 8, 4, 1, 0], dtype=np.int64)
    return z, y
