"""Helpers shared by the GPU parity tests.

Error measure (reported per case, gated by the tolerance written in each test):
    max_abs  = max |gpu - ref|
    norm_err = max |gpu - ref| / max(1, max |ref|)
with ``ref`` the fp64 oracle evaluated on the same fp32 inputs.  When the
environment variable XM_PARITY_REPORT names a file, every check appends one
JSON line with these figures.
"""

import json
import os

import numpy as np

# Tolerances on norm_err (fp32 device path vs fp64 oracle).
TOL_SS = 1e-4
TOL_M3 = 1e-4
TOL_GDN2 = 2e-4


def to_dev(x, device="cuda"):
    import torch
    if x is None:
        return None
    return torch.from_numpy(np.require(x, requirements=["C", "W"])).to(device)


def errors(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if got.size == 0:
        return 0.0, 0.0, 0.0
    d = np.abs(got - ref)
    assert np.all(np.isfinite(got)), "non-finite output"
    max_abs = float(d.max())
    ref_inf = float(np.abs(ref).max())
    return max_abs, max_abs / max(1.0, ref_inf), ref_inf


def check(name, got, ref, tol):
    max_abs, norm_err, ref_inf = errors(got, ref)
    path = os.environ.get("XM_PARITY_REPORT")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(dict(case=name, max_abs=max_abs, norm_err=norm_err, ref_inf=ref_inf, tol=tol)) + "\n")
    assert norm_err <= tol, f"{name}: max_abs={max_abs:.3e} norm_err={norm_err:.3e} > tol={tol:.1e}"
    return max_abs, norm_err
