"""SelectiveScanFn's sequence-parallel form (SelectiveScanSegKernel) on the GPU
vs the fp64 oracle, through the C ABI.

The form splits each channel's sequence into 16-token segments, scans them at
once and composes their affine maps (the reference's SSMScanOp and chunk
prefix, selective_scan_common.h:148-153, :170-182).  It is selected
automatically when the single-pass kernel would have fewer channel blocks
than CUs and the sequence is at least 256 tokens long; the ``ss_split``
override forces it (2) or the single pass (1).  Covered: every state layout
(dstate 1 to 256), constant and variable B/C, groups, ragged and unaligned
sequences (the guarded loads), carries across blocks, the last state, 16-bit
data, the automatic selection, and a 65536-token sequence."""

import numpy as np
import pytest

from oracle import cref
from parity import TOL_GPU, TOL_SS, check, to_dev
from xmetai_onnx_plugins import last_launches, selective_scan_fn, workloads as W

pytestmark = pytest.mark.gpu

KEYS = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")


def run_gpu(inp, softplus=True, state=False):
    import torch
    r = selective_scan_fn(*(to_dev(inp[k]) for k in KEYS), delta_softplus=softplus, return_last_state=state)
    torch.cuda.synchronize()
    if state:
        return r[0].cpu().numpy(), r[1].cpu().numpy()
    return r.cpu().numpy()


def run_ref(inp, softplus=True, state=False):
    return cref.selective_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], None,
                               inp["delta_bias"], delta_softplus=softplus, dtype=np.float64, return_state=state)


def seg_launched():
    return any(k.startswith("SelectiveScanSegKernel") for k in last_launches())


CASES = {
    # dstate across the lane layouts: (4,1) (8,1) (8,2) (16,2) (16,4) (16,8) (16,16)
    "n1_l300": W.SelectiveScanShape(2, 5, 300, 1),
    "n3_l37_ragged": W.SelectiveScanShape(2, 9, 37, 3),
    "n4_l512": W.SelectiveScanShape(1, 6, 512, 4),
    "n8_l260": W.SelectiveScanShape(2, 7, 260, 8),
    "n16_l512": W.SelectiveScanShape(1, 12, 512, 16),
    "n16_l1": W.SelectiveScanShape(3, 4, 1, 16),
    "n16_l5": W.SelectiveScanShape(1, 4, 5, 16),
    "n24_l300": W.SelectiveScanShape(1, 5, 300, 24),
    "n32_l257": W.SelectiveScanShape(1, 6, 257, 32),
    "n64_l700": W.SelectiveScanShape(1, 5, 700, 64),
    "n100_l333": W.SelectiveScanShape(1, 3, 333, 100),
    "n128_l512": W.SelectiveScanShape(1, 3, 512, 128),
    "n256_l300": W.SelectiveScanShape(1, 2, 300, 256),
    # B/C forms and groups
    "n16_groups2": W.SelectiveScanShape(2, 16, 400, 16, groups=2),
    "n64_groups4": W.SelectiveScanShape(2, 8, 300, 64, groups=4),
    "n16_const_b": W.SelectiveScanShape(1, 6, 300, 16, b_var=False),
    "n16_const_c": W.SelectiveScanShape(1, 6, 300, 16, c_var=False),
    "n16_const_bc": W.SelectiveScanShape(1, 6, 300, 16, b_var=False, c_var=False),
    "n64_const_bc": W.SelectiveScanShape(1, 4, 300, 64, b_var=False, c_var=False),
    "n16_no_d_z_bias": W.SelectiveScanShape(1, 6, 300, 16, has_d=False, has_z=False, has_bias=False),
    "n16_no_softplus": W.SelectiveScanShape(1, 6, 300, 16, delta_softplus=False),
    # carries across blocks (512 tokens per block at dstate 16, 256 at 32..256)
    "n16_l513": W.SelectiveScanShape(1, 4, 513, 16),
    "n16_l2050": W.SelectiveScanShape(1, 4, 2050, 16),
    "n16_l4096": W.SelectiveScanShape(2, 3, 4096, 16),
    "n64_l1030": W.SelectiveScanShape(1, 3, 1030, 64),
    "n256_l520": W.SelectiveScanShape(1, 2, 520, 256),
}


def _inputs(s, seed):
    inp = W.selective_scan_inputs(s, seed=seed)
    if not s.delta_softplus:
        # keep delta' = delta + bias >= 0 so exp(delta' A) stays a decay
        inp["delta"] = np.abs(inp["delta"]) * np.float32(0.1)
        inp["delta_bias"] = np.zeros_like(inp["delta_bias"])
    return inp


@pytest.mark.parametrize("name", sorted(CASES))
def test_seg_parity(name, override):
    s = CASES[name]
    inp = _inputs(s, seed=11)
    override("ss_split", 2)
    y = run_gpu(inp, s.delta_softplus)
    assert seg_launched(), last_launches()
    check(f"selective_scan_seg/{name}", y, run_ref(inp, s.delta_softplus), TOL_SS)


@pytest.mark.parametrize("name", ["n1_l300", "n16_l2050", "n16_const_bc", "n64_l1030", "n256_l520", "n3_l37_ragged"])
def test_seg_last_state(name, override):
    s = CASES[name]
    inp = _inputs(s, seed=12)
    override("ss_split", 2)
    y, h = run_gpu(inp, s.delta_softplus, state=True)
    assert seg_launched()
    ref_y, ref_h = run_ref(inp, s.delta_softplus, state=True)
    check(f"selective_scan_seg_state/{name}/y", y, ref_y, TOL_SS)
    check(f"selective_scan_seg_state/{name}/h", h, ref_h, TOL_SS)
    np.testing.assert_array_equal(y, run_gpu(inp, s.delta_softplus))   # the state write leaves y alone


def test_seg_unaligned_inputs(override):
    # Offsets of one float take the guarded loads; results must not change.
    import torch
    s = W.SelectiveScanShape(1, 6, 300, 16)
    inp = W.selective_scan_inputs(s, seed=13)

    def shifted(x):
        buf = torch.empty(x.size + 1, dtype=torch.float32, device="cuda")
        t = buf[1:].view(x.shape)
        t.copy_(torch.from_numpy(x))
        return t
    override("ss_split", 2)
    y = selective_scan_fn(shifted(inp["u"]), shifted(inp["delta"]), to_dev(inp["A"]), shifted(inp["B"]),
                          shifted(inp["C"]), to_dev(inp["D"]), to_dev(inp["z"]), to_dev(inp["delta_bias"]),
                          delta_softplus=True)
    assert seg_launched()
    check("selective_scan_seg/unaligned", y.cpu().numpy(), run_ref(inp), TOL_SS)


def test_seg_selected_for_few_channels(override):
    """The CPU-runnable configuration (1 x 256 x 512, dstate 16: 8 channel
    blocks) takes the split form by itself; the single pass agrees."""
    override("ss_split", 0)
    inp = W.selective_scan_inputs(W.SS_CPU, seed=0)
    y = run_gpu(inp)
    assert seg_launched(), last_launches()
    check("selective_scan_seg/auto_b1_d256_l512_n16", y, run_ref(inp), TOL_SS)
    override("ss_split", 1)
    y1 = run_gpu(inp)
    assert not seg_launched()
    check("selective_scan_seg/auto_vs_single_pass", y, y1, TOL_GPU)


def test_seg_not_selected_for_many_channels(override):
    # 8 x 2048 channels at dstate 16: 512 channel blocks of 32
    override("ss_split", 0)
    inp = W.selective_scan_inputs(W.SelectiveScanShape(8, 2048, 256, 16), seed=0)
    run_gpu(inp)
    assert not seg_launched(), last_launches()


def test_seg_long_sequence():
    """1 x 64 x 65536, dstate 16: 128 blocks of 512 tokens per channel, every
    carry in VGPRs; the whole output and the last state against the oracle."""
    s = W.SelectiveScanShape(1, 64, 65536, 16)
    inp = W.selective_scan_inputs(s, seed=14)
    y, h = run_gpu(inp, state=True)
    assert seg_launched(), last_launches()
    ref_y, ref_h = run_ref(inp, state=True)
    check("selective_scan_seg/b1_d64_l65536_n16", y, ref_y, TOL_SS)
    check("selective_scan_seg/b1_d64_l65536_n16/h", h, ref_h, TOL_SS)


@pytest.mark.parametrize("fmt", ["float16", "bfloat16"])
@pytest.mark.parametrize("shape", [W.SelectiveScanShape(1, 8, 600, 16), W.SelectiveScanShape(1, 5, 301, 16),
                                   W.SelectiveScanShape(1, 4, 300, 64, b_var=False)],
                         ids=["n16_l600", "n16_l301_ragged", "n64_const_b"])
def test_seg_16bit(fmt, shape, override):
    """16-bit data: the fp64 oracle on the 16-bit-rounded inputs; y within one
    unit of the 16-bit format plus 1e-5 (as for the single pass)."""
    import torch
    tdt = getattr(torch, fmt)
    mant = {"float16": 10, "bfloat16": 7}[fmt]
    inp = W.selective_scan_inputs(shape, seed=15)
    dev, rounded = {}, {}
    for k in KEYS:
        x = inp[k]
        if x is None:
            dev[k] = rounded[k] = None
            continue
        t = to_dev(x)
        if k in ("u", "delta", "z") or (k in ("B", "C") and x.ndim >= 3):
            t = t.to(tdt)
            rounded[k] = t.float().cpu().numpy()
        else:
            rounded[k] = x
        dev[k] = t
    override("ss_split", 2)
    y, h = selective_scan_fn(*(dev[k] for k in KEYS), delta_softplus=True, return_last_state=True)
    torch.cuda.synchronize()
    assert seg_launched()
    assert y.dtype == tdt
    ref_y, ref_h = run_ref(rounded, state=True)
    got = y.float().cpu().numpy().astype(np.float64)
    spacing = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref_y), 2.0 ** -14))) - mant)
    err = np.abs(got - ref_y)
    assert np.all(err <= spacing + 1e-5), float((err / (spacing + 1e-5)).max())
    check(f"selective_scan_seg_16bit/{fmt}/h", h.cpu().numpy(), ref_h, TOL_SS)


@pytest.mark.parametrize("L", [4, 5])
def test_seg_softplus_range(L, override):
    """delta' = softplus(delta + bias) over [-80, 80] read out exactly through
    the split form's staging (A = 0, u one-hot at token 0, B = 1, C one-hot on
    state 0): x > 20 returns x bit for bit, below within a few ulp."""
    import torch
    D, N = 64, 16
    x = np.linspace(-80, 80, D, dtype=np.float32)
    x[:3] = [20.0, np.nextafter(np.float32(20), np.float32(21)), 20.5]
    dev = torch.device("cuda")
    delta = torch.zeros(1, D, L, device=dev)
    delta[0, :, 0] = torch.from_numpy(x).to(dev)
    u = torch.zeros(1, D, L, device=dev)
    u[0, :, 0] = 1.0
    A = torch.zeros(D, N, device=dev)
    Bm = torch.ones(1, 1, N, L, device=dev)
    Cm = torch.zeros(1, 1, N, L, device=dev)
    Cm[:, :, 0] = 1.0
    override("ss_split", 2)
    y = selective_scan_fn(u, delta, A, Bm, Cm, torch.zeros(D, device=dev), None, torch.zeros(D, device=dev),
                          delta_softplus=True)
    assert seg_launched()
    got = y[0, :, 0].cpu().numpy().astype(np.float64)
    xd = x.astype(np.float64)
    big = x > 20
    assert np.array_equal(got[big], xd[big])
    ref = np.log1p(np.exp(xd[~big]))
    bound = (8 + 2 * np.abs(xd[~big])) * 2.0 ** -24 * ref
    assert np.all(np.abs(got[~big] - ref) <= bound)
