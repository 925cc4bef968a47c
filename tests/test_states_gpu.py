"""State outputs (and Mamba-3's state inputs) on the GPU vs the fp64 oracle,
through the C ABI.

SelectiveScanFn with return_last_state=1 writes the scan state after the last
token, [B,D,N]; GatedDeltaNet2Fn with output_final_state=1 writes the state
after the last token, [B,H,K,V] (initial_state's layout).  Both attributes
are rejected by the reference's ORT kernels (selective_scan_fn_ort.cpp:52-55,
gated_deltanet2_fn_ort.cpp:49-51); here they are a widening served by the
``*_forward_states`` entry points.  Checked: the state against the oracle's,
output 0 unchanged bit for bit by the extra write, every kernel variant
(lane layouts, key tiles, rows per column, the LDS-state path with its chunk
carry), empty sequences, and chaining (two calls joined through the state
equal one call).
"""

import numpy as np
import pytest

from oracle import cref
from parity import TOL_GPU, TOL_GDN2, TOL_M3, TOL_SS, check, to_dev
from xmetai_onnx_plugins import gated_deltanet2_fn, mamba3_siso_fn, selective_scan_fn, workloads as W
import xmetai_onnx_plugins as xp

pytestmark = pytest.mark.gpu

SS_KEYS = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
GDN_KEYS = ("q", "k", "v", "g", "beta", "w", "initial_state")


# ---------------------------------------------------------------------------
# SelectiveScanFn last_state
# ---------------------------------------------------------------------------

def ss_gpu(inp, softplus=True, state=True):
    import torch
    r = selective_scan_fn(*(to_dev(inp[k]) for k in SS_KEYS), delta_softplus=softplus, return_last_state=state)
    torch.cuda.synchronize()
    if state:
        return r[0].cpu().numpy(), r[1].cpu().numpy()
    return r.cpu().numpy()


def ss_ref(inp, softplus=True):
    return cref.selective_scan(*(inp[k] for k in SS_KEYS), delta_softplus=softplus, dtype=np.float64,
                               return_state=True)


SS_CASES = {
    "n1": W.SelectiveScanShape(2, 40, 64, 1),
    "n3_ragged_l37": W.SelectiveScanShape(2, 33, 37, 3),
    "n16_groups2": W.SelectiveScanShape(2, 96, 64, 16, groups=2),
    "n16_const_bc": W.SelectiveScanShape(1, 70, 48, 16, b_var=False, c_var=False),
    "n16_l1": W.SelectiveScanShape(3, 64, 1, 16),
    "n16_l2050": W.SelectiveScanShape(1, 16, 2050, 16),
    "n64_groups4": W.SelectiveScanShape(2, 64, 40, 64, groups=4),
    "n100": W.SelectiveScanShape(1, 20, 33, 100),
    "n256": W.SelectiveScanShape(1, 17, 24, 256),
}


@pytest.mark.parametrize("name", sorted(SS_CASES))
def test_ss_last_state_parity(name):
    s = SS_CASES[name]
    inp = W.selective_scan_inputs(s, seed=4)
    y, h = ss_gpu(inp)
    ref_y, ref_h = ss_ref(inp)
    assert h.shape == (s.batch, s.dim, s.dstate)
    check(f"selective_scan_state/{name}/y", y, ref_y, TOL_SS)
    check(f"selective_scan_state/{name}/h", h, ref_h, TOL_SS)
    np.testing.assert_array_equal(y, ss_gpu(inp, state=False))   # the state write leaves y alone


@pytest.mark.parametrize("lpc", [4, 8, 16])
def test_ss_last_state_lane_layouts(lpc, override):
    s = W.SelectiveScanShape(2, 70, 45, 16)
    inp = W.selective_scan_inputs(s, seed=5)
    override("ss_lpc", lpc)
    y, h = ss_gpu(inp)
    ref_y, ref_h = ss_ref(inp)
    check(f"selective_scan_state/lpc{lpc}/y", y, ref_y, TOL_SS)
    check(f"selective_scan_state/lpc{lpc}/h", h, ref_h, TOL_SS)


def test_ss_last_state_of_an_empty_sequence_is_zero():
    import torch
    s = W.SelectiveScanShape(2, 8, 0, 4)
    inp = W.selective_scan_inputs(s, seed=0)
    args = [to_dev(inp[k]) for k in SS_KEYS]
    args[0] = torch.zeros((2, 8, 0), device="cuda")
    args[1] = torch.zeros((2, 8, 0), device="cuda")
    y, h = selective_scan_fn(*args, delta_softplus=True, return_last_state=True)
    torch.cuda.synchronize()
    assert y.shape == (2, 8, 0) and h.shape == (2, 8, 4)
    assert torch.count_nonzero(h).item() == 0


# ---------------------------------------------------------------------------
# GatedDeltaNet2Fn final_state
# ---------------------------------------------------------------------------

def gdn_gpu(inp, s, state=True):
    import torch
    r = gated_deltanet2_fn(*(to_dev(inp[k]) for k in GDN_KEYS), scale=s.scale, use_qk_l2norm_in_kernel=s.l2norm,
                           output_final_state=state)
    torch.cuda.synchronize()
    if state:
        return r[0].cpu().numpy(), r[1].cpu().numpy()
    return r.cpu().numpy()


def gdn_ref(inp, s):
    return cref.gated_deltanet2(*(inp[k] for k in GDN_KEYS), scale=s.scale, use_qk_l2norm=s.l2norm,
                                dtype=np.float64, return_state=True)


S = W.GatedDeltaNet2Shape
GDN_CASES = {
    "k1_v1": S(1, 9, 2, 1, 1),
    "t1_single_token": S(2, 1, 3, 64, 32),
    "t3_shorter_than_block": S(1, 3, 2, 128, 40, per_key_gates=True),
    "k17_v15_partial": S(2, 20, 2, 17, 15),
    "k32_v33_nos0": S(1, 40, 2, 32, 33, initial_state=False),
    "k128_v65_partial_wave": S(2, 64, 4, 128, 65),
    "k200_v40": S(1, 17, 2, 200, 40),
    "k257_two_rows": S(1, 21, 2, 257, 20),
    "k512_v7_perkey": S(1, 12, 1, 512, 7, per_key_gates=True),
    "k600_v33_lds_path": S(2, 40, 2, 600, 33),
    "t1500_lds_carry": S(1, 1500, 1, 600, 16),
    "k1024_lds_path_perkey": S(1, 12, 1, 1024, 7, per_key_gates=True),
    "t4100_three_windows": S(1, 4100, 2, 64, 24),
    "k448_t2100_window_carry": S(1, 2100, 1, 448, 12, per_key_gates=True),
    "k2100_tile_store": S(1, 30, 2, 2100, 20),
    "k4096_t1100_tile_store_carry": S(1, 1100, 1, 4096, 16),
}


@pytest.mark.parametrize("name", sorted(GDN_CASES))
def test_gdn2_final_state_parity(name):
    s = GDN_CASES[name]
    inp = W.gated_deltanet2_inputs(s, seed=6)
    o, st = gdn_gpu(inp, s)
    ref_o, ref_st = gdn_ref(inp, s)
    assert st.shape == (s.batch, s.nheads, s.dk, s.dv)
    check(f"gated_deltanet2_state/{name}/o", o, ref_o, TOL_GDN2)
    check(f"gated_deltanet2_state/{name}/S", st, ref_st, TOL_GDN2)
    np.testing.assert_array_equal(o, gdn_gpu(inp, s, state=False))   # the state write leaves o alone


@pytest.mark.parametrize("shape,mode", [((1, 1500, 2, 96, 40, True), 2), ((2, 700, 1, 320, 24, False), 2),
                                        ((1, 90, 1, 33, 17, True), 2), ((1, 1500, 2, 96, 40, True), 3),
                                        ((2, 700, 1, 256, 24, False), 3), ((1, 90, 1, 40, 17, True), 3)])
def test_gdn2_final_state_sequence_split(shape, mode, override):
    """The final state of a sequence-split call (gdn2_split = 2: up to four
    equal segments; 3: two unequal segments, the second two tiles per
    workgroup): the combine kernel's last step, from the initial state or
    zeros."""
    b, t, h, k, v, s0 = shape
    s = S(b, t, h, k, v, initial_state=s0)
    inp = W.gated_deltanet2_inputs(s, seed=8)
    override("gdn2_split", mode)
    o, st = gdn_gpu(inp, s)
    kernel = "Gdn2ChunkSplit2Kernel" if mode == 3 else "Gdn2ChunkSplitKernel"
    assert any(x.startswith(kernel) for x in xp.last_launches()), xp.last_launches()
    ref_o, ref_st = gdn_ref(inp, s)
    check(f"gated_deltanet2_state/split{mode}_{b}_{t}_{h}_{k}_{v}/o", o, ref_o, TOL_GDN2)
    check(f"gated_deltanet2_state/split{mode}_{b}_{t}_{h}_{k}_{v}/S", st, ref_st, TOL_GDN2)


@pytest.mark.parametrize("name", ["t4100_three_windows", "k448_t2100_window_carry"])
def test_gdn2_final_state_windows_of_128_chunks(name, override):
    """The final state after 128-chunk windows (gdn2_windowed), the state
    carried between them."""
    s = GDN_CASES[name]
    inp = W.gated_deltanet2_inputs(s, seed=6)
    override("gdn2_windowed", 1)
    o, st = gdn_gpu(inp, s)
    ref_o, ref_st = gdn_ref(inp, s)
    check(f"gated_deltanet2_state/{name}/windows128/o", o, ref_o, TOL_GDN2)
    check(f"gated_deltanet2_state/{name}/windows128/S", st, ref_st, TOL_GDN2)


@pytest.mark.parametrize("rows", [1, 2, 4])
def test_gdn2_final_state_rows_per_column(rows, override):
    s = S(2, 37, 3, 64, 40)
    inp = W.gated_deltanet2_inputs(s, seed=7)
    override("gdn2_path", 1)   # the sequential kernel's column layouts
    override("gdn2_rows", rows)
    o, st = gdn_gpu(inp, s)
    ref_o, ref_st = gdn_ref(inp, s)
    check(f"gated_deltanet2_state/rows{rows}/o", o, ref_o, TOL_GDN2)
    check(f"gated_deltanet2_state/rows{rows}/S", st, ref_st, TOL_GDN2)


@pytest.mark.parametrize("shape,split", [((2, 300, 4, 128, 128), 123), ((1, 700, 2, 384, 16), 333),
                                         ((1, 1100, 2, 600, 24), 1030)])
def test_gdn2_final_state_chains(shape, split):
    """Tokens [0, split) then [split, T) started from the first call's final
    state give the outputs and final state of one call over [0, T)."""
    import torch
    s = S(*shape)
    inp = W.gated_deltanet2_inputs(s, seed=8)
    dev = {k: to_dev(v) for k, v in inp.items()}
    kw = dict(scale=s.scale, use_qk_l2norm_in_kernel=s.l2norm, output_final_state=True)
    o, st = gated_deltanet2_fn(*(dev[k] for k in GDN_KEYS), **kw)
    part = lambda a, b: [dev[k][:, a:b].contiguous() for k in GDN_KEYS[:-1]]
    o1, st1 = gated_deltanet2_fn(*part(0, split), dev["initial_state"], **kw)
    o2, st2 = gated_deltanet2_fn(*part(split, s.seqlen), st1, **kw)
    torch.cuda.synchronize()
    whole = o.cpu().numpy()
    chained = torch.cat([o1, o2], dim=1).cpu().numpy()
    # the same arithmetic in the same order, with the state passing through fp32 memory
    check(f"gated_deltanet2_state/chain_{split}/o", chained, whole, TOL_GPU)
    check(f"gated_deltanet2_state/chain_{split}/S", st2.cpu().numpy(), st.cpu().numpy(), TOL_GPU)


# ---------------------------------------------------------------------------
# Mamba3SisoFn states (ssm [B,H,P,N], angle [B,H,A], k [B,H,N], v [B,H,P])
# ---------------------------------------------------------------------------

M3_KEYS = ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")
M3 = W.Mamba3SisoShape
M3_STATE_NAMES = ("ssm", "angle", "k", "v")


def m3_states_for(s, seed):
    rng = np.random.default_rng(seed)
    B, H, P, N, A = s.batch, s.nheads, s.headdim, s.dstate, s.a
    return ((0.3 * rng.standard_normal((B, H, P, N))).astype(np.float32),
            rng.uniform(0.0, 6.28, (B, H, A)).astype(np.float32),
            (rng.standard_normal((B, H, N)) * N ** -0.5).astype(np.float32),
            rng.standard_normal((B, H, P)).astype(np.float32))


def m3_gpu(inp, ins=None, state=True):
    import torch
    r = mamba3_siso_fn(*(to_dev(inp[k]) for k in M3_KEYS),
                       input_states=None if ins is None else tuple(to_dev(x) for x in ins),
                       return_final_states=state)
    torch.cuda.synchronize()
    if state:
        return r[0].cpu().numpy(), [x.cpu().numpy() for x in r[1]]
    return r.cpu().numpy()


def m3_ref(inp, ins=None):
    return cref.mamba3_siso(*(inp[k] for k in M3_KEYS), dtype=np.float64, input_states=ins, return_state=True)


def check_m3_states(tag, got, ref, tol):
    for g, r, nm in zip(got, ref, M3_STATE_NAMES):
        if nm == "angle":   # compare on the circle: a wrap near 0 / 2 pi may fall either side
            two_pi = 2.0 * float(np.float32(np.pi))
            g = r + (np.mod(g - r + two_pi / 2, two_pi) - two_pi / 2)
        check(f"{tag}/{nm}", g, r, tol)


M3_CASES = {
    "t1_n16": M3(2, 1, 2, 8, 16),
    "n8_p7": M3(2, 17, 3, 7, 8),
    "n64_p33_hq1_z": M3(1, 33, 4, 33, 64, nheads_qk=1, has_z=True),
    "n128_a7": M3(1, 40, 2, 64, 128, angles=7),
    "n512_p64": M3(1, 35, 2, 64, 512),
    "n1100_p16_a300_z": M3(1, 30, 2, 16, 1100, angles=300, has_z=True),   # three key-block launches
    "n130_padded": M3(1, 25, 2, 20, 130),
    "n256": M3(1, 21, 2, 24, 256),
    "p65_rowblocks_t70": M3(2, 70, 2, 65, 32),
}


@pytest.mark.parametrize("with_inputs", [False, True])
@pytest.mark.parametrize("name", sorted(M3_CASES))
def test_m3_states_parity(name, with_inputs, m3_path):
    s = M3_CASES[name]
    inp = W.mamba3_siso_inputs(s, seed=9)
    ins = m3_states_for(s, 10) if with_inputs else None
    y, st = m3_gpu(inp, ins)
    ry, rst = m3_ref(inp, ins)
    assert [x.shape for x in st] == [x.shape for x in rst]
    check(f"mamba3_state/{name}/{with_inputs}/y", y, ry, TOL_M3)
    check_m3_states(f"mamba3_state/{name}/{with_inputs}", st, rst, TOL_M3)
    np.testing.assert_array_equal(y, m3_gpu(inp, ins, state=False))   # the state writes leave y alone


@pytest.mark.parametrize("shape,split", [((2, 100, 4, 16, 32), 37), ((1, 70, 2, 65, 128), 32),
                                         ((1, 45, 2, 20, 256), 1)])
def test_m3_states_chain(shape, split, m3_path):
    """Tokens [0, split) then [split, T) continued from the first call's states
    give the outputs and states of one call over [0, T)."""
    import torch
    s = M3(*shape, has_z=True)
    inp = W.mamba3_siso_inputs(s, seed=11)
    dev = {k: to_dev(v) for k, v in inp.items() if v is not None}
    T = s.seqlen

    def part(a, b):
        out = []
        for k in M3_KEYS:
            x = dev.get(k)
            if x is None or k in ("Q_bias", "K_bias", "D"):
                out.append(x)
            elif k in ("ADT", "DT", "Trap"):
                out.append(x[:, :, a:b].contiguous())
            else:
                out.append(x[:, a:b].contiguous())
        return out

    y, st = mamba3_siso_fn(*part(0, T), return_final_states=True)
    y1, st1 = mamba3_siso_fn(*part(0, split), return_final_states=True)
    y2, st2 = mamba3_siso_fn(*part(split, T), input_states=st1, return_final_states=True)
    torch.cuda.synchronize()
    check(f"mamba3_state/chain_{split}/y", torch.cat([y1, y2], dim=1).cpu().numpy(), y.cpu().numpy(), TOL_GPU)
    check_m3_states(f"mamba3_state/chain_{split}", [x.cpu().numpy() for x in st2], [x.cpu().numpy() for x in st], TOL_GPU)


@pytest.mark.parametrize("name", ["t3_shorter_than_block", "k32_v33_nos0", "k128_v65_partial_wave", "k200_v40",
                                  "t4100_three_windows"])
def test_gdn2_final_state_two_column_tiles(name, override):
    """Final states of both column tiles of a two-tile workgroup (gdn2_ct)."""
    s = GDN_CASES[name]
    inp = W.gated_deltanet2_inputs(s, seed=6)
    override("gdn2_ct", 2)
    override("gdn2_split", 1)
    o, st = gdn_gpu(inp, s)
    ref_o, ref_st = gdn_ref(inp, s)
    check(f"gated_deltanet2_state/{name}/ct2/o", o, ref_o, TOL_GDN2)
    check(f"gated_deltanet2_state/{name}/ct2/S", st, ref_st, TOL_GDN2)
