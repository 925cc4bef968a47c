"""Helpers shared by the GPU parity tests.

Error measures (reported per case, gated by the tolerances below), with
``ref`` the fp64 oracle evaluated on the same fp32 inputs:

    max_abs  = max |gpu - ref|
    norm_err = max |gpu - ref| / max |ref|                              (whole tensor)
    row_err  = max over rows r of max_r |gpu - ref| / max(max_r |ref|, 1e-3 max |ref|)

Both are relative to the output's own scale (GDN-2 outputs are ~1e-3, so an
absolute bound would be loose).  A row is a line along the last axis (the
value columns of one token and head, or the tokens of one selective-scan
channel).  ``row_err`` is the per-element gate
|gpu - ref| <= tol_row * max(max |ref| of the row, 1e-3 max |ref|): an output
whose magnitude grows along the sequence (GatedDeltaNet2Fn without the L2
norm) cannot hide an error in its small early rows behind the large late ones.
When the environment variable XM_PARITY_REPORT names a file, every check
appends one JSON line with these figures and the kernel overrides in force.

Gates (measured worst on MI355X over the whole GPU suite, every kernel path,
times about 10):

    op        worst norm_err   worst row_err   gate norm / row
    SS        3.4e-7           1.3e-6          3e-6 / 2e-5
    Mamba-3   5.8e-7           4.2e-6          6e-6 / 4e-5
    GDN-2     4.1e-7           8.1e-6          8e-6 / 8e-5
    GPU vs GPU (chained calls, packed vs plain, chunked vs token-by-token):
              5.0e-7           5.5e-6          5e-6 / 6e-5

Ill-conditioned cases (an exploding GDN-2 state without the L2 norm, growing
or hard-reset decays, thousands of large angle steps) lose accuracy in any
fp32 evaluation order.  For them the test also runs the oracle in fp32 with
the reference's operation order and each bound becomes max(gate, 8 x that
fp32 error): the device must be about as accurate as the reference's own
fp32 recurrence.  Measured (device / fp32 order, row_err): GDN-2 without L2
norm 3.2e-6 / 1.7e-6; Mamba-3 growth 6.5e-6 / 4.4e-6; long angle runs
3.7e-6 / 6.3e-6; GDN-2 hard reset (-200) 8.2e-7 / 1.3e-6.
"""

import json
import os
from typing import NamedTuple

import numpy as np


class Gate(NamedTuple):
    norm: float   # bound on norm_err
    row: float    # bound on row_err


# fp32 device path vs the fp64 oracle, per operator
TOL_SS = Gate(3e-6, 2e-5)
TOL_M3 = Gate(6e-6, 4e-5)
TOL_GDN2 = Gate(8e-6, 8e-5)
TOL_GPU = Gate(5e-6, 6e-5)   # one device path against another
FP32_FACTOR = 8.0            # ill-conditioned cases: multiple of the fp32-order oracle's error


def to_dev(x, device="cuda"):
    import torch
    if x is None:
        return None
    return torch.from_numpy(np.require(x, requirements=["C", "W"])).to(device)


def errors(got, ref):
    """(max_abs, norm_err, ref_inf, row_err) of `got` against `ref`."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if got.size == 0:
        return 0.0, 0.0, 0.0, 0.0
    assert np.all(np.isfinite(got)), "non-finite output"
    d = np.abs(got - ref)
    max_abs = float(d.max())
    ref_inf = float(np.abs(ref).max())
    scale = ref_inf if ref_inf > 0 else 1.0
    # a last axis of length 1 (a one-state SS state, a one-token output) makes
    # every element its own row: the tensor is then one row
    rows = ref.shape[-1] if ref.ndim and ref.shape[-1] > 1 else ref.size
    d2 = d.reshape(-1, rows)
    r2 = np.abs(ref).reshape(-1, rows)
    row_err = float((d2.max(axis=1) / np.maximum(1e-3 * scale, r2.max(axis=1))).max())
    return max_abs, max_abs / scale, ref_inf, row_err


def _overrides():
    try:
        import xmetai_onnx_plugins as xp
        from xmetai_onnx_plugins import _capi
    except ImportError:
        return {}
    if xp._lib is None:
        return {}
    return {k: v for k in _capi.KERNEL_OVERRIDES if (v := xp.get_kernel_override(k)) != 0}


def check(name, got, ref, gate, ref32=None):
    """Gates norm_err <= gate.norm and row_err <= gate.row (a plain number
    bounds both).  With ``ref32`` (the oracle in fp32, reference operation
    order) each bound is raised to FP32_FACTOR times that evaluation's own
    error against ``ref``."""
    if not isinstance(gate, Gate):
        gate = Gate(float(gate), float(gate))
    tol, tol_row = gate
    extra = {}
    if ref32 is not None:
        _, n32, _, r32 = errors(ref32, ref)
        tol = max(tol, FP32_FACTOR * n32)
        tol_row = max(tol_row, FP32_FACTOR * r32)
        extra = dict(fp32_norm_err=n32, fp32_row_err=r32)
    max_abs, norm_err, ref_inf, row_err = errors(got, ref)
    path = os.environ.get("XM_PARITY_REPORT")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(dict(case=name, max_abs=max_abs, norm_err=norm_err, row_err=row_err, ref_inf=ref_inf,
                                    tol=tol, tol_row=tol_row, overrides=_overrides(), **extra)) + "\n")
    assert norm_err <= tol, f"{name}: max_abs={max_abs:.3e} norm_err={norm_err:.3e} > tol={tol:.1e}"
    assert row_err <= tol_row, f"{name}: row_err={row_err:.3e} > tol_row={tol_row:.1e} (max_abs={max_abs:.3e})"
    return max_abs, norm_err
