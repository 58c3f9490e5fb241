"""Loads the known-answer fixtures of tests/golden/ as torch tensors."""

from __future__ import annotations

import glob
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16}


def names(kind: str) -> list[str]:
    out = []
    for path in sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))):
        with np.load(path) as z:
            if str(z["kind"]) == kind:
                out.append(os.path.splitext(os.path.basename(path))[0])
    return out


def load(name: str, device="cpu") -> dict:
    with np.load(os.path.join(GOLDEN, f"{name}.npz")) as z:
        dt = DTYPES[str(z["dtype"])]
        out = {"kind": str(z["kind"]), "dtype": dt}
        for key in z.files:
            if key in ("kind", "dtype"):
                continue
            arr = z[key]
            if arr.dtype == np.int16:
                out[key] = torch.from_numpy(arr.copy()).view(dt).to(device)
            elif key in ("scale",):
                out[key] = float(arr)
            elif key in ("out",) or key.endswith("_out"):
                out[key] = torch.from_numpy(arr.copy())
            else:
                out[key] = torch.from_numpy(arr.copy()).to(device)
        return out
