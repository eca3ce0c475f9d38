"""Writes the small regression fixtures under tests/golden/ from the fp64 oracle.

The reference holds no golden vectors or fixture files for this path (its
tests compare against its loop oracle at run time), so these fixtures are
produced by this repository's float64 oracle, itself pinned by the closed
form, finite differences and invariants in tests/test_oracle_*.py.  They are
data (inputs and expected outputs), regenerated with:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import wkv4, wkv7  # noqa: E402

OUT = Path(__file__).resolve().parent


def wkv4_cases():
    cases = {}
    for name, (b, t, c, seed) in {
        "b2t16c8": (2, 16, 8, 0),
        "b1t1c5": (1, 1, 5, 1),
        "b3t33c70": (3, 33, 70, 2),
    }.items():
        k, v, td, tf, gy = wkv4.make_inputs(b, t, c, seed=seed, dtype=torch.float64)
        td, tf = td.double(), tf.double()
        y, gk, gv, gtd, gtf = wkv4.autograd_grads(k, v, td, tf, gy)
        for key, val in dict(k=k, v=v, td=td, tf=tf, gy=gy, y=y, gk=gk, gv=gv, gtd=gtd, gtf=gtf).items():
            cases[f"{name}__{key}"] = val.numpy()
    return cases


def wkv7_cases():
    cases = {}
    r, w, k, v, a, b = wkv7.make_inputs(1, 12, 2, 64, seed=3, dtype=torch.float64)
    y, s = wkv7.wkv7_loop(r, w, k, v, a, b)
    gy = torch.randn(y.shape, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    _, _, dr, dw, dk, dv, da, db, _ = wkv7.wkv7_autograd_grads(r, w, k, v, a, b, None, gy)
    fields = dict(r=r, w=w, k=k, v=v, a=a, b=b, y=y, s=s, gy=gy, dr=dr, dw=dw, dk=dk, dv=dv, da=da, db=db)
    for key, val in fields.items():
        cases[f"b1t12h2__{key}"] = val.numpy()
    return cases


if __name__ == "__main__":
    np.savez_compressed(OUT / "wkv4_small.npz", **wkv4_cases())
    np.savez_compressed(OUT / "wkv7_small.npz", **wkv7_cases())
    print("wrote", OUT / "wkv4_small.npz", OUT / "wkv7_small.npz")
