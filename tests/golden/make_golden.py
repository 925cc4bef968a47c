"""Writes the small golden fixtures under tests/golden/ (inputs + fp64 outputs).

    python tests/golden/make_golden.py

The outputs come from the fp64 oracle (oracle/xm_oracle.c), after both oracle
restatements (C and NumPy) are checked to agree on them.  The reference
publishes no vectors for these operators, so these fixtures freeze the pinned
oracle: tests/test_golden.py re-derives them on the CPU, and the GPU tests
compare the device path against them.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "xmetai-onnx-plugins_amd"))

from oracle import cref, numpy_ref  # noqa: E402
from xmetai_onnx_plugins import workloads as W  # noqa: E402

FIXTURES = {
    "selective_scan_small": ("ss", W.SelectiveScanShape(2, 8, 33, 16), 11),
    "selective_scan_groups_const_c": ("ss", W.SelectiveScanShape(1, 6, 20, 5, groups=2, c_var=False), 12),
    "gated_deltanet2_small": ("gdn2", W.GatedDeltaNet2Shape(1, 40, 2, 32, 8, per_key_gates=True), 13),
    "gated_deltanet2_widek": ("gdn2", W.GatedDeltaNet2Shape(1, 6, 1, 260, 4), 14),
    "mamba3_siso_small": ("m3", W.Mamba3SisoShape(1, 24, 2, 8, 16, angles=6, has_z=True), 15),
}


def compute(kind, s, inp):
    if kind == "ss":
        args = [inp[k] for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")]
        a = cref.selective_scan(*args, delta_softplus=s.delta_softplus, dtype=np.float64)
        b = numpy_ref.selective_scan(*args, delta_softplus=s.delta_softplus, dtype=np.float64)
        attrs = dict(delta_softplus=int(s.delta_softplus))
    elif kind == "gdn2":
        args = [inp[k] for k in ("q", "k", "v", "g", "beta", "w", "initial_state")]
        a = cref.gated_deltanet2(*args, scale=s.scale, use_qk_l2norm=s.l2norm, dtype=np.float64)
        b = numpy_ref.gated_deltanet2(*args, scale=s.scale, use_qk_l2norm=s.l2norm, dtype=np.float64)
        attrs = dict(scale=np.float32(s.scale), use_qk_l2norm_in_kernel=int(s.l2norm))
    else:
        args = [inp[k] for k in ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")]
        a = cref.mamba3_siso(*args, dtype=np.float64)
        b = numpy_ref.mamba3_siso(*args, dtype=np.float64)
        attrs = dict(has_d=int(s.has_d), has_z=int(s.has_z))
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)
    return a, attrs


def main():
    for name, (kind, s, seed) in FIXTURES.items():
        gen = {"ss": W.selective_scan_inputs, "gdn2": W.gated_deltanet2_inputs, "m3": W.mamba3_siso_inputs}[kind]
        inp = gen(s, seed=seed)
        out, attrs = compute(kind, s, inp)
        arrays = {f"in_{k}": v for k, v in inp.items() if v is not None}
        arrays.update({f"attr_{k}": np.asarray(v) for k, v in attrs.items()})
        arrays["out"] = out
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
