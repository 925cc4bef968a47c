"""PreparedCall (``prepare=True``): the argument blocks of one operator call
built once and re-enqueued.  Every call must equal the plain function's
result bit for bit (same C entry point, same kernels, same buffers), also
with the state outputs, and after the inputs change in place."""

import numpy as np
import pytest

from parity import to_dev
from xmetai_onnx_plugins import gated_deltanet2_fn, mamba3_siso_fn, selective_scan_fn, workloads as W

pytestmark = pytest.mark.gpu


def test_prepared_selective_scan():
    import torch
    inp = W.selective_scan_inputs(W.SelectiveScanShape(2, 40, 300, 16), seed=21)
    keys = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
    d = {k: to_dev(inp[k]) for k in keys}
    args = [d[k] for k in keys]
    call = selective_scan_fn(*args, delta_softplus=True, prepare=True)
    for _ in range(3):
        y = call()
        assert y is call.out
        assert torch.equal(y, selective_scan_fn(*args, delta_softplus=True))
    d["u"].mul_(0.5)   # same buffers, new contents
    assert torch.equal(call(), selective_scan_fn(*args, delta_softplus=True))
    st = selective_scan_fn(*args, delta_softplus=True, return_last_state=True, prepare=True)
    y, h = st()
    y0, h0 = selective_scan_fn(*args, delta_softplus=True, return_last_state=True)
    assert torch.equal(y, y0) and torch.equal(h, h0)


def test_prepared_gated_deltanet2():
    import torch
    s = W.GatedDeltaNet2Shape(batch=2, seqlen=200, nheads=3, dk=64, dv=48, initial_state=True)
    inp = W.gated_deltanet2_inputs(s, seed=22)
    keys = ("q", "k", "v", "g", "beta", "w", "initial_state")
    args = [to_dev(inp[k]) for k in keys]
    call = gated_deltanet2_fn(*args, scale=s.scale, output_final_state=True, prepare=True)
    o0, f0 = gated_deltanet2_fn(*args, scale=s.scale, output_final_state=True)
    for _ in range(2):
        o, f = call()
        assert torch.equal(o, o0) and torch.equal(f, f0)


def test_prepared_mamba3_siso():
    import torch
    s = W.Mamba3SisoShape(batch=2, seqlen=100, nheads=4, headdim=32, dstate=32, angles=16, has_d=True, has_z=True)
    inp = W.mamba3_siso_inputs(s, seed=23)
    keys = ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")
    args = [to_dev(inp[k]) for k in keys]
    call = mamba3_siso_fn(*args, prepare=True)
    y0 = mamba3_siso_fn(*args)
    for _ in range(2):
        assert torch.equal(call(), y0)
