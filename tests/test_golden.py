"""Golden fixtures (tests/golden/*.npz): the oracle must reproduce them on
the CPU, and the device path must match them within the stated tolerance."""

import glob
import os

import numpy as np
import pytest

from oracle import cref, numpy_ref
from parity import TOL_GDN2, TOL_M3, TOL_SS, check, to_dev

HERE = os.path.dirname(os.path.abspath(__file__))
FILES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))

SS_KEYS = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
GDN_KEYS = ("q", "k", "v", "g", "beta", "w", "initial_state")
M3_KEYS = ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")


def load(path):
    with np.load(path, allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    name = os.path.basename(path)[:-4]
    inputs = {k[3:]: v for k, v in d.items() if k.startswith("in_")}
    attrs = {k[5:]: v.item() for k, v in d.items() if k.startswith("attr_")}
    return name, inputs, attrs, d["out"]


def _args(inputs, keys):
    return [inputs.get(k) for k in keys]


def test_fixtures_present():
    assert len(FILES) >= 5


@pytest.mark.parametrize("path", FILES, ids=lambda p: os.path.basename(p))
@pytest.mark.parametrize("impl", [cref, numpy_ref], ids=["c", "numpy"])
def test_oracle_reproduces_golden(path, impl):
    name, inp, attrs, out = load(path)
    if name.startswith("selective_scan"):
        y = impl.selective_scan(*_args(inp, SS_KEYS), delta_softplus=bool(attrs["delta_softplus"]), dtype=np.float64)
    elif name.startswith("gated_deltanet2"):
        y = impl.gated_deltanet2(*_args(inp, GDN_KEYS), scale=attrs["scale"],
                                 use_qk_l2norm=bool(attrs["use_qk_l2norm_in_kernel"]), dtype=np.float64)
    else:
        y = impl.mamba3_siso(*_args(inp, M3_KEYS), dtype=np.float64)
    np.testing.assert_allclose(y, out, rtol=1e-12, atol=1e-13)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=lambda p: os.path.basename(p))
def test_device_matches_golden(path):
    import torch
    import xmetai_onnx_plugins as xp
    name, inp, attrs, out = load(path)
    if name.startswith("selective_scan"):
        y = xp.selective_scan_fn(*(to_dev(x) for x in _args(inp, SS_KEYS)), delta_softplus=bool(attrs["delta_softplus"]))
        tol = TOL_SS
    elif name.startswith("gated_deltanet2"):
        y = xp.gated_deltanet2_fn(*(to_dev(x) for x in _args(inp, GDN_KEYS)), scale=attrs["scale"],
                                  use_qk_l2norm_in_kernel=bool(attrs["use_qk_l2norm_in_kernel"]))
        tol = TOL_GDN2
    else:
        y = xp.mamba3_siso_fn(*(to_dev(x) for x in _args(inp, M3_KEYS)), has_d=bool(attrs["has_d"]),
                              has_z=bool(attrs["has_z"]))
        tol = TOL_M3
    torch.cuda.synchronize()
    check(f"golden/{name}", y.cpu().numpy(), out, tol)
