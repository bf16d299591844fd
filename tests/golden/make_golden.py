"""Write the golden vectors of tests/golden/ with the reference's own CPU path.

The reference CPU extension (src/cpu/fw_cpu.cpp) is compiled into oracle/_ref by
oracle/build_oracle.py; this script calls its fw_loss_grad (src/cpu/fwcpp.py:21-23) on seeded
inputs and stores inputs and outputs as data:

    z [R, C] float32, y [R] int64, scale          inputs (reduced slices of each configuration and
                                                 hand-made edge rows); golden_f64.npz holds
                                                 float64 cases, keys prefixed by the case name
    L [R] float64, kappa [R] int64               per-row loss and support size
    g_rows, g_cols [nnz] int64, g_vals [nnz] f32 the non-zeros of scale * gradient

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "fast-familywise-loss_amd")]

import torch  # noqa: E402

import fwloss_data  # noqa: E402
import oracle  # noqa: E402

CASES = {
    "cfg1": dict(cfg="cfg1", N=256, seed=11),
    "cfg2": dict(cfg="cfg2", N=24, seed=12),
    "cfg3": dict(cfg="cfg3", N=256, seed=13),
    "cfg4": dict(cfg="cfg4", N=3, seed=14),
    "cfg5": dict(cfg="cfg5", N=1, seed=15),
}


def run_ref(ref, z, y, scale, vals_dtype=np.float32):
    L, G, k = ref.fw_loss_grad(torch.from_numpy(z), torch.from_numpy(y), float(scale), 2 ** 62, 100000, True)
    G = G.numpy()
    rows, cols = np.nonzero(G)
    return dict(L=L.numpy().astype(np.float64), kappa=k.numpy().astype(np.int64), g_rows=rows.astype(np.int64),
                g_cols=cols.astype(np.int64), g_vals=G[rows, cols].astype(vals_dtype))


def main():
    ref = oracle.load_ref()
    if ref is None:
        raise SystemExit("oracle/_ref is not built (python oracle/build_oracle.py --ref)")
    for name, c in CASES.items():
        z, y = fwloss_data.make(c["cfg"], N=c["N"], seed=c["seed"])
        scale = 1.0 / z.shape[0]
        out = run_ref(ref, z, y, scale)
        np.savez_compressed(os.path.join(HERE, f"golden_{name}.npz"), z=z, y=y, scale=np.float64(scale), **out)
        print(name, z.shape, "kappa", out["kappa"].min(), out["kappa"].max(), flush=True)
    z, y = fwloss_data.edge_rows()
    out = run_ref(ref, z, y, 1.0)
    np.savez_compressed(os.path.join(HERE, "golden_edges.npz"), z=z, y=y, scale=np.float64(1.0), **out)
    print("edges", z.shape, "kappa", out["kappa"], flush=True)
    # float64 logits (the reference's run_generic<double>, fw_cpu.cpp:697-703)
    parts = {}
    for name, z in f64_cases().items():
        y = np.random.default_rng(len(name)).integers(0, z.shape[1], z.shape[0]).astype(np.int64)
        scale = 1.0 / z.shape[0]
        out = run_ref(ref, z, y, scale, vals_dtype=np.float64)
        for k, v in dict(z=z, y=y, scale=np.float64(scale), **out).items():
            parts[f"{name}_{k}"] = v
        print("f64", name, z.shape, "kappa", out["kappa"].min(), out["kappa"].max(), flush=True)
    np.savez_compressed(os.path.join(HERE, "golden_f64.npz"), **parts)


def f64_cases():
    rng = np.random.default_rng(64)
    gauss = rng.standard_normal((48, 1000))
    ties = 0.5 * rng.integers(-8, 9, (128, 100)).astype(np.float64)
    wide = rng.standard_normal((8, 5001)) * 3.0
    flat = np.tile(np.linspace(0.0, 1e-3, 700), (4, 1))     # hundreds of entries within 1 of the max
    return {"gauss": gauss, "ties": ties, "wide": wide, "flat": flat}


if __name__ == "__main__":
    main()
