"""SelectiveScanFn with float16 / bfloat16 data on the GPU, through the C ABI.

A widening: the reference has half and bfloat16 kernel instantiations
(selective_scan_fwd_fp16.cu:9-10, selective_scan_fwd_bf16.cu) that its
fp32-only host cannot reach (ort_common.h:90-92).  u, delta, z and variable
B/C are 16-bit, A, D, delta_bias and constant B/C fp32, the arithmetic fp32,
and y is the fp32 result rounded to the 16-bit type.  The fp64 oracle runs on
the same 16-bit-rounded inputs; y must then be within one unit in the last
place of the 16-bit format (rounding of a value whose fp32 computation is off
by ~1e-6 can land on either side of a midpoint), plus 1e-5 absolute for the
fp32 arithmetic.  The fp32 last state is held to the fp32 tolerance.
"""

import numpy as np
import pytest

from oracle import cref
from parity import TOL_SS, check, to_dev
from xmetai_onnx_plugins import selective_scan_fn, workloads as W

pytestmark = pytest.mark.gpu

KEYS = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
DATA = ("u", "delta", "z")
MANT = {"float16": 10, "bfloat16": 7}   # explicit mantissa bits


def ulp(x, mant):
    """The spacing of the format at |x| (normal range; floored at the smallest normal's)."""
    ax = np.maximum(np.abs(x), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(ax)) - mant)


@pytest.mark.parametrize("fmt", ["float16", "bfloat16"])
@pytest.mark.parametrize("shape", [W.SelectiveScanShape(2, 64, 64, 16), W.SelectiveScanShape(1, 40, 37, 16),
                                   W.SelectiveScanShape(2, 96, 64, 16, groups=2),
                                   W.SelectiveScanShape(1, 70, 48, 16, b_var=False, c_var=False),
                                   W.SelectiveScanShape(1, 20, 33, 64), W.SelectiveScanShape(1, 17, 24, 256)],
                         ids=["n16", "n16_l37_ragged", "n16_groups2", "n16_const_bc", "n64_l33", "n256"])
def test_ss_16bit_parity(fmt, shape):
    import torch
    tdt = getattr(torch, fmt)
    inp = W.selective_scan_inputs(shape, seed=17)
    dev, rounded = {}, {}
    for k in KEYS:
        x = inp[k]
        if x is None:
            dev[k] = None
            rounded[k] = None
            continue
        data = k in DATA or (k in ("B", "C") and x.ndim >= 3)
        t = to_dev(x)
        if data:
            t = t.to(tdt)
            rounded[k] = t.float().cpu().numpy()   # exactly the 16-bit values
        else:
            rounded[k] = x
        dev[k] = t
    y, h = selective_scan_fn(*(dev[k] for k in KEYS), delta_softplus=True, return_last_state=True)
    torch.cuda.synchronize()
    assert y.dtype == tdt and h.dtype == torch.float32
    ref_y, ref_h = cref.selective_scan(*(rounded[k] for k in KEYS), delta_softplus=True, dtype=np.float64,
                                       return_state=True)
    got = y.float().cpu().numpy()
    err = np.abs(got - ref_y)
    bound = ulp(ref_y, MANT[fmt]) + 1e-5
    assert np.all(err <= bound), f"{fmt}: worst {float(np.max(err / bound)):.3f} of the bound"
    check(f"selective_scan_{fmt}/h", h.cpu().numpy(), ref_h, TOL_SS)


@pytest.mark.parametrize("fmt", ["float16", "bfloat16"])
def test_ss_16bit_matches_fp32_call_on_the_same_values(fmt):
    """A 16-bit call and an fp32 call on the same (16-bit) values share the fp32
    arithmetic, so y16 is y32 rounded to nearest even: compared with torch's
    own float -> 16-bit conversion, a truncating or biased rounding would
    differ on about half the elements.  Allowed: a rare 1-unit difference
    where the two fp32 results straddle a midpoint."""
    import torch
    tdt = getattr(torch, fmt)
    s = W.SelectiveScanShape(2, 128, 256, 16)
    inp = W.selective_scan_inputs(s, seed=18)
    dev16 = {k: (to_dev(v).to(tdt) if k in ("u", "delta", "z", "B", "C") else to_dev(v)) if v is not None else None
             for k, v in inp.items()}
    dev32 = {k: (v.float() if v is not None else None) for k, v in dev16.items()}
    y16 = selective_scan_fn(*(dev16[k] for k in KEYS), delta_softplus=True)
    y32 = selective_scan_fn(*(dev32[k] for k in KEYS), delta_softplus=True)
    torch.cuda.synchronize()
    a = y16.float().cpu().numpy()
    b = y32.to(tdt).float().cpu().numpy()
    assert np.all(np.abs(a - b) <= ulp(b, MANT[fmt])), float(np.max(np.abs(a - b) / ulp(b, MANT[fmt])))
    assert np.mean(a != b) <= 1e-3, f"{fmt}: {np.mean(a != b):.4f} of y differ from the rounded fp32 result"
