"""The ONNX Runtime custom-op layer run end to end on the GPU through the ONNX
Runtime API double (tests/ort_double): for each device operator a node is
created from its attributes and Compute runs on device tensors bound as an
ONNX Runtime session binds them: the execution provider's compute stream, and
scratch from KernelContext_GetScratchBuffer, handed back through the context
allocator.  The outputs must equal, bit for bit, those of the direct C ABI call
on the same tensors (the layer adds no arithmetic), and match the fp64 oracle.
Covered: SelectiveScanFn in fp32, fp16 and bf16 (descriptor chosen by the
data type) with the last state; GatedDeltaNet2Fn with the initial and final
state, packed sequences (input 7) and the trailing optional input omitted;
Mamba3SisoFn with D, Z, the input states (inputs 11-14) and the four final
states; nodes with exactly the reference's inputs and outputs (the optional
tails absent).

Reference: selective_scan_fn_ort.cpp:58-150, gated_deltanet2_fn_ort.cpp:66-142,
mamba3_siso_fn_ort.cpp:61-145 (Compute), ort_common.h:74-101 (tensor views)."""

import numpy as np
import pytest

import ortd
from oracle import cref
from parity import TOL_GDN2, TOL_M3, TOL_SS, check, to_dev
import xmetai_onnx_plugins as xp
from xmetai_onnx_plugins import workloads as W

pytestmark = pytest.mark.gpu


def stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def scratch():
    import torch
    return torch.empty(256 << 20, dtype=torch.uint8, device="cuda")


def like(shape, dtype=None):
    import torch
    return torch.full((int(np.prod(shape)),), float("nan"), dtype=dtype or torch.float32, device="cuda")


def done(*xs):
    import torch
    torch.cuda.synchronize()
    return [x.float().cpu().numpy() for x in xs]


SS_KEYS = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")


def test_selective_scan_fp32_with_state():
    s = W.SelectiveScanShape(2, 64, 300, 16)
    inp = W.selective_scan_inputs(s, seed=31)
    dev = [to_dev(inp[k]) for k in SS_KEYS]
    (y, h), _ = ortd.run("SelectiveScanFn", dev, [like((2, 64, 300)), like((2, 64, 16))],
                         ints={"delta_softplus": 1, "return_last_state": 1}, stream=stream())
    assert tuple(y.shape) == (2, 64, 300) and tuple(h.shape) == (2, 64, 16)
    y, h = done(y, h)
    dy, dh = xp.selective_scan_fn(*dev, delta_softplus=True, return_last_state=True)
    dy, dh = done(dy, dh)
    np.testing.assert_array_equal(y, dy)
    np.testing.assert_array_equal(h, dh)
    ry, rh = cref.selective_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], None,
                                 inp["delta_bias"], delta_softplus=True, dtype=np.float64, return_state=True)
    check("ort/selective_scan/y", y, ry, TOL_SS)
    check("ort/selective_scan/state", h, rh, TOL_SS)


@pytest.mark.parametrize("fmt", ["float16", "bfloat16"])
def test_selective_scan_16bit_descriptor(fmt):
    import torch
    tdt = getattr(torch, fmt)
    s = W.SelectiveScanShape(1, 32, 200, 16)
    inp = W.selective_scan_inputs(s, seed=32)
    dev = []
    for k in SS_KEYS:
        t = to_dev(inp[k])
        if k in ("u", "delta", "z", "B", "C"):
            t = t.to(tdt)
        dev.append(t)
    (y,), _ = ortd.run("SelectiveScanFn", dev, [like((1, 32, 200), tdt)], ints={"delta_softplus": 1},
                       stream=stream())
    assert y.dtype == tdt
    dy = xp.selective_scan_fn(*dev, delta_softplus=True)
    y, dy = done(y, dy)
    np.testing.assert_array_equal(y, dy)


GDN_KEYS = ("q", "k", "v", "g", "beta", "w", "initial_state")


def test_gated_deltanet2_with_states_and_scratch():
    s = W.GatedDeltaNet2Shape(2, 150, 3, 64, 32)
    inp = W.gated_deltanet2_inputs(s, seed=33)
    dev = [to_dev(inp[k]) for k in GDN_KEYS]
    (o, st), (peak, frees) = ortd.run("GatedDeltaNet2Fn", dev, [like((2, 150, 3, 32)), like((2, 3, 64, 32))],
                                      ints={"output_final_state": 1, "use_qk_l2norm_in_kernel": 1},
                                      floats={"scale": s.scale}, stream=stream(), scratch=scratch())
    assert peak > 0 and frees > 0   # the chunked path's scratch, through the context's buffers
    o, st = done(o, st)
    do, dst = xp.gated_deltanet2_fn(*dev, scale=s.scale, output_final_state=True)
    do, dst = done(do, dst)
    np.testing.assert_array_equal(o, do)
    np.testing.assert_array_equal(st, dst)
    ro, rs = cref.gated_deltanet2(*(inp[k] for k in GDN_KEYS), scale=s.scale, use_qk_l2norm=True, dtype=np.float64,
                                  return_state=True)
    check("ort/gated_deltanet2/o", o, ro, TOL_GDN2)
    check("ort/gated_deltanet2/state", st, rs, TOL_GDN2)


def test_gated_deltanet2_defaults_and_omitted_optional_input():
    """No attributes (scale 1, L2 norm on) and input 7 bound as missing, as
    ONNX Runtime passes an absent trailing optional input."""
    s = W.GatedDeltaNet2Shape(1, 40, 2, 32, 16)
    inp = W.gated_deltanet2_inputs(s, seed=34)
    dev = [to_dev(inp[k]) for k in GDN_KEYS]
    (o,), _ = ortd.run("GatedDeltaNet2Fn", dev + [None], [like((1, 40, 2, 16))], stream=stream(), scratch=scratch())
    do = xp.gated_deltanet2_fn(*dev, scale=1.0)
    o, do = done(o, do)
    np.testing.assert_array_equal(o, do)


def test_gated_deltanet2_packed():
    import torch
    lens = [50, 0, 77, 13]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T, N = int(cu[-1]), len(lens)
    s = W.GatedDeltaNet2Shape(1, T, 2, 64, 24, initial_state=False)
    inp = W.gated_deltanet2_inputs(s, seed=35)
    s0 = (0.05 * np.random.default_rng(36).standard_normal((N, 2, 64, 24))).astype(np.float32)
    dev = [to_dev(inp[k]) for k in GDN_KEYS[:6]] + [to_dev(s0), torch.from_numpy(cu).cuda()]
    (o, st), _ = ortd.run("GatedDeltaNet2Fn", dev, [like((1, T, 2, 24)), like((N, 2, 64, 24))],
                          ints={"has_cu_seqlens": 1, "output_final_state": 1}, floats={"scale": s.scale},
                          stream=stream(), scratch=scratch())
    do, dst = xp.gated_deltanet2_fn(*dev[:7], scale=s.scale, output_final_state=True, cu_seqlens=dev[7])
    o, st, do, dst = done(o, st, do, dst)
    np.testing.assert_array_equal(o, do)
    np.testing.assert_array_equal(st, dst)
    for n in range(N):
        a, e = int(cu[n]), int(cu[n + 1])
        if a == e:
            np.testing.assert_array_equal(st[n], s0[n])
            continue
        part = [np.ascontiguousarray(inp[k][:, a:e]) for k in GDN_KEYS[:6]]
        ro, rs = cref.gated_deltanet2(*part, s0[n:n + 1], scale=s.scale, use_qk_l2norm=True, dtype=np.float64,
                                      return_state=True)
        check(f"ort/gated_deltanet2/packed{n}/o", o[:, a:e], ro, TOL_GDN2)
        check(f"ort/gated_deltanet2/packed{n}/state", st[n:n + 1], rs, TOL_GDN2)


M3_KEYS = ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")


def test_mamba3_with_input_and_final_states():
    s = W.Mamba3SisoShape(1, 70, 2, 16, 32, has_z=True)
    inp = W.mamba3_siso_inputs(s, seed=37)
    dev = [to_dev(inp[k]) for k in M3_KEYS]
    B, H, P, N, A = 1, 2, 16, 32, s.a
    rng = np.random.default_rng(38)
    ins_states = [(0.1 * rng.standard_normal(sh)).astype(np.float32)
                  for sh in ((B, H, P, N), (B, H, A), (B, H, N), (B, H, P))]
    dstates = [to_dev(x) for x in ins_states]
    outs = [like((B, 70, H, P)), like((B, H, P, N)), like((B, H, A)), like((B, H, N)), like((B, H, P))]
    res, _ = ortd.run("Mamba3SisoFn", dev + dstates, outs,
                      ints={"chunk_size": 64, "has_d": 1, "has_z": 1, "return_final_states": 1,
                            "has_input_states": 1}, stream=stream(), scratch=scratch())
    assert [tuple(r.shape) for r in res] == [(B, 70, H, P), (B, H, P, N), (B, H, A), (B, H, N), (B, H, P)]
    got = done(*res)
    dy, dst = xp.mamba3_siso_fn(*dev, input_states=dstates, return_final_states=True)
    want = done(dy, *dst)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    ry, rst = cref.mamba3_siso(*(inp[k] for k in M3_KEYS), dtype=np.float64, input_states=ins_states,
                               return_state=True)
    check("ort/mamba3/y", got[0], ry, TOL_M3)
    for i, name in enumerate(("ssm", "angle", "k", "v")):
        g, r = got[1 + i], rst[i]
        if name == "angle":   # on the circle: a wrap near 0 / 2 pi may fall either side
            two_pi = 2.0 * float(np.float32(np.pi))
            g = r + (np.mod(g - r + two_pi / 2, two_pi) - two_pi / 2)
        check(f"ort/mamba3/{name}", g, r, TOL_M3)


def test_reference_arity_nodes():
    """Nodes with exactly the reference's inputs and outputs (GatedDeltaNet2Fn
    7 inputs and 1 output, gated_deltanet2_fn_ort.cpp; Mamba3SisoFn 11 inputs
    and 1 output, mamba3_siso_fn_ort.cpp): the optional tails this layer
    declares beyond them (cu_seqlens, the states) read as absent, and the
    outputs equal the direct C ABI call bit for bit."""
    s = W.GatedDeltaNet2Shape(2, 50, 3, 48, 20)
    inp = W.gated_deltanet2_inputs(s, seed=41)
    dev = [to_dev(inp[k]) for k in GDN_KEYS]
    assert len(dev) == 7
    (o,), _ = ortd.run("GatedDeltaNet2Fn", dev, [like((2, 50, 3, 20))], floats={"scale": s.scale},
                       stream=stream(), scratch=scratch())
    o, do = done(o, xp.gated_deltanet2_fn(*dev, scale=s.scale))
    np.testing.assert_array_equal(o, do)

    m = W.Mamba3SisoShape(1, 40, 2, 16, 32, has_z=True)
    minp = W.mamba3_siso_inputs(m, seed=42)
    mdev = [to_dev(minp[k]) for k in M3_KEYS]
    assert len(mdev) == 11
    (y,), _ = ortd.run("Mamba3SisoFn", mdev, [like((1, 40, 2, 16))],
                       ints={"chunk_size": 64, "has_d": 1, "has_z": 1}, stream=stream(), scratch=scratch())
    y, dy = done(y, xp.mamba3_siso_fn(*mdev))
    np.testing.assert_array_equal(y, dy)
