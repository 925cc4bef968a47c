"""Packed sequences (cu_seqlens) on the GPU, through the C ABI.

GatedDeltaNet2Fn and Mamba3SisoFn with has_cu_seqlens=1 (a widening: the
reference rejects it, gated_deltanet2_fn_ort.cpp:55-57, mamba3_siso_fn_ort.cpp:
56-58) take N sequences packed along one row of tokens, with one state per
sequence.  Each packed call is checked against the fp64 oracle run on every
sequence by itself, with that sequence's initial state: outputs and final
states.  Covered: empty and one-token sequences, lengths that end inside a
token block, every GDN-2 key layout up to headdim_k 512 on the chunked path
(global-chunk windows, a sequence's state carried between windows) and on the
sequential kernel, sequences spanning several windows, runs of empty
sequences, Mamba-3 with and without input states.
"""

import numpy as np
import pytest

from oracle import cref
from parity import TOL_GPU, TOL_GDN2, TOL_M3, check, to_dev
from xmetai_onnx_plugins import gated_deltanet2_fn, mamba3_siso_fn, workloads as W

pytestmark = pytest.mark.gpu

GDN_KEYS = ("q", "k", "v", "g", "beta", "w")
M3_KEYS = ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")


def offsets(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)


def cu_dev(lengths):
    import torch
    return torch.from_numpy(offsets(lengths)).to("cuda")


@pytest.fixture(params=["chunk", "seq"])
def gdn2_path(request, override):
    """GatedDeltaNet2Fn kernel under test: the chunked MFMA path (default) or
    the sequential fused kernel (gdn2_path override 1)."""
    override("gdn2_path", 1 if request.param == "seq" else 0)
    return request.param


def gdn2_packed_check(lengths, H, dk, dv, with_state, path, seed, tag):
    """Runs one packed call and checks every sequence against the oracle run
    on it alone."""
    import torch
    import xmetai_onnx_plugins as xp
    T, N = sum(lengths), len(lengths)
    s = W.GatedDeltaNet2Shape(1, T, H, dk, dv, initial_state=False)
    inp = W.gated_deltanet2_inputs(s, seed=seed)
    rng = np.random.default_rng(seed + 1)
    s0 = (0.05 * rng.standard_normal((N, H, dk, dv))).astype(np.float32) if with_state else None
    o, st = gated_deltanet2_fn(*(to_dev(inp[k]) for k in GDN_KEYS), None if s0 is None else to_dev(s0),
                               scale=s.scale, use_qk_l2norm_in_kernel=s.l2norm, output_final_state=True,
                               cu_seqlens=cu_dev(lengths))
    torch.cuda.synchronize()
    launched = xp.last_launches()
    if path == "chunk":
        assert any(k.startswith("Gdn2ChunkRecurKernel") and ",1>" in k for k in launched), launched
    else:
        assert any(k.startswith("Gdn2FusedKernel") for k in launched), launched
    o, st = o.cpu().numpy(), st.cpu().numpy()
    assert o.shape == (1, T, H, dv) and st.shape == (N, H, dk, dv)
    cu = offsets(lengths)
    for n in range(N):
        lo, hi = cu[n], cu[n + 1]
        init = s0[n:n + 1] if s0 is not None else np.zeros((1, H, dk, dv), np.float32)
        if hi == lo:   # an empty sequence passes its state through
            np.testing.assert_array_equal(st[n], init[0])
            continue
        part = [np.ascontiguousarray(inp[k][:, lo:hi]) for k in GDN_KEYS]
        ro, rs = cref.gated_deltanet2(*part, init, scale=s.scale, use_qk_l2norm=s.l2norm, dtype=np.float64,
                                      return_state=True)
        check(f"{tag}/{path}/seq{n}/o", o[:, lo:hi], ro, TOL_GDN2)
        check(f"{tag}/{path}/seq{n}/S", st[n:n + 1], rs, TOL_GDN2)


# ---------------------------------------------------------------------------
# GatedDeltaNet2Fn
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dk,dv", [(16, 8), (64, 40), (128, 65), (320, 24), (512, 16)])
@pytest.mark.parametrize("with_state", [False, True])
def test_gdn2_packed_matches_per_sequence(dk, dv, with_state, gdn2_path):
    gdn2_packed_check([37, 0, 1, 16, 50], 2, dk, dv, with_state, gdn2_path, 12, f"gdn2_packed/{dk}x{dv}")


@pytest.mark.parametrize("dk,dv", [(64, 32), (128, 128), (256, 20)])
def test_gdn2_packed_long_sequences(dk, dv):
    """Sequences of 1500-3000 tokens with empty and short ones between them
    (one window over every chunk)."""
    gdn2_packed_check([3000, 0, 1500, 17, 2100, 5], 2, dk, dv, True, "chunk", 31, f"gdn2_packed_long/{dk}x{dv}")


def test_gdn2_packed_across_windows():
    """50007 tokens at headdim_k 512: one window over every chunk would take
    641 MB of prepared blocks, so the row is stepped in windows of 128 chunks
    per sequence; the 30000- and 20000-token sequences carry their states
    through 15 and 10 windows."""
    gdn2_packed_check([30000, 7, 20000], 2, 512, 16, True, "chunk", 33, "gdn2_packed_windows")


def test_gdn2_packed_many_sequences_with_empties():
    """300 sequences of 0 to 40 tokens, a third of them empty, runs of empties
    included: more sequences than a window has slots, found through the chunk
    offsets; every empty sequence passes its initial state through."""
    rng = np.random.default_rng(41)
    lengths = [int(x) for x in rng.integers(1, 41, 300)]
    for i in rng.choice(300, 100, replace=False):
        lengths[i] = 0
    lengths[10:30] = [0] * 20
    gdn2_packed_check(lengths, 2, 64, 24, True, "chunk", 42, "gdn2_packed_many")


def test_gdn2_packed_one_sequence_equals_unpacked():
    """One sequence covering the whole row: the same outputs as the plain call
    (which takes the chunked path at dk = 128) within the tolerance."""
    import torch
    s = W.GatedDeltaNet2Shape(1, 300, 4, 128, 128)
    inp = W.gated_deltanet2_inputs(s, seed=14)
    args = [to_dev(inp[k]) for k in GDN_KEYS] + [to_dev(inp["initial_state"])]
    kw = dict(scale=s.scale, use_qk_l2norm_in_kernel=s.l2norm, output_final_state=True)
    o1, s1 = gated_deltanet2_fn(*args, **kw)
    o2, s2 = gated_deltanet2_fn(*args, cu_seqlens=cu_dev([300]), **kw)
    torch.cuda.synchronize()
    check("gdn2_packed/one/o", o2.cpu().numpy(), o1.cpu().numpy(), TOL_GPU)
    check("gdn2_packed/one/S", s2.cpu().numpy(), s1.cpu().numpy(), TOL_GPU)


# ---------------------------------------------------------------------------
# Mamba3SisoFn
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n_qk,p_dim,hq", [(16, 8, 1), (64, 33, 2), (128, 64, 2), (256, 24, 2), (768, 16, 2)])
@pytest.mark.parametrize("with_states", [False, True])
def test_m3_packed_matches_per_sequence(n_qk, p_dim, hq, with_states, m3_path):
    import torch
    lengths = [45, 1, 0, 33, 70]
    T, H, N = sum(lengths), 2, len(lengths)
    s = W.Mamba3SisoShape(1, T, H, p_dim, n_qk, nheads_qk=hq, has_z=True)
    inp = W.mamba3_siso_inputs(s, seed=15)
    A = s.a
    rng = np.random.default_rng(16)
    ins = None
    if with_states:
        ins = ((0.3 * rng.standard_normal((N, H, p_dim, n_qk))).astype(np.float32),
               rng.uniform(0, 6.28, (N, H, A)).astype(np.float32),
               (rng.standard_normal((N, H, n_qk)) * n_qk ** -0.5).astype(np.float32),
               rng.standard_normal((N, H, p_dim)).astype(np.float32))
    y, st = mamba3_siso_fn(*(to_dev(inp[k]) for k in M3_KEYS),
                           input_states=None if ins is None else tuple(to_dev(x) for x in ins),
                           return_final_states=True, cu_seqlens=cu_dev(lengths))
    torch.cuda.synchronize()
    y, st = y.cpu().numpy(), [x.cpu().numpy() for x in st]
    assert y.shape == (1, T, H, p_dim) and st[0].shape == (N, H, p_dim, n_qk)
    cu = offsets(lengths)
    two_pi = 2.0 * float(np.float32(np.pi))
    for n in range(N):
        lo, hi = cu[n], cu[n + 1]
        init = tuple(x[n:n + 1] for x in ins) if ins is not None else None
        if hi == lo:   # an empty sequence passes its states through (zeros without input states)
            for got, x in zip(st, init or [None] * 4):
                np.testing.assert_array_equal(got[n], x[0] if x is not None else 0.0)
            continue
        part = {}
        for k in M3_KEYS:
            x = inp[k]
            if x is None or k in ("Q_bias", "K_bias", "D"):
                part[k] = x
            elif k in ("ADT", "DT", "Trap"):
                part[k] = np.ascontiguousarray(x[:, :, lo:hi])
            else:
                part[k] = np.ascontiguousarray(x[:, lo:hi])
        ry, rst = cref.mamba3_siso(*(part[k] for k in M3_KEYS), dtype=np.float64, input_states=init,
                                   return_state=True)
        tag = f"m3_packed/{n_qk}x{p_dim}/seq{n}"
        check(f"{tag}/y", y[:, lo:hi], ry, TOL_M3)
        for g, r, nm in zip(st, rst, ("ssm", "angle", "k", "v")):
            g = g[n:n + 1]
            if nm == "angle":
                g = r + (np.mod(g - r + two_pi / 2, two_pi) - two_pi / 2)
            check(f"{tag}/{nm}", g, r, TOL_M3)


# ---------------------------------------------------------------------------
# Token rows that no sequence covers
# ---------------------------------------------------------------------------

def _covered(cu, T):
    """Tokens covered by the sequences [lo_b, hi_b) (lo_b = clamp(cu[b]), hi_b =
    clamp(max(cu[b + 1], lo_b)), the kernels' reading of the offsets)."""
    cov = np.zeros(T, bool)
    ranges = []
    for b in range(len(cu) - 1):
        lo = min(max(cu[b], 0), T)
        hi = min(max(cu[b + 1], lo), T)
        cov[lo:hi] = True
        ranges.append((lo, hi))
    return cov, ranges


GAP_CASES = {"head_and_tail_gaps": ([3, 20, 20, 50], 64), "non_monotone": ([10, 12, 2, 4], 16)}


@pytest.mark.parametrize("case", sorted(GAP_CASES))
def test_gdn2_packed_uncovered_rows_are_zero(case, gdn2_path):
    """Offsets that leave token rows outside every sequence (cu[0] > 0,
    cu[N] < T, or non-monotone offsets): those rows of the output are zeros
    (the buffer holds NaN before the call); the covered rows match the oracle
    per sequence."""
    import torch
    cu, T = GAP_CASES[case]
    H, dk, dv = 2, 32, 16
    s = W.GatedDeltaNet2Shape(1, T, H, dk, dv, initial_state=False)
    inp = W.gated_deltanet2_inputs(s, seed=51)
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda")
    call = gated_deltanet2_fn(*(to_dev(inp[k]) for k in GDN_KEYS), None, scale=s.scale, cu_seqlens=cu_t,
                              prepare=True)
    call.out.fill_(float("nan"))
    o = call().cpu().numpy()
    cov, ranges = _covered(cu, T)
    assert np.all(o[:, ~cov] == 0.0)
    for n, (lo, hi) in enumerate(ranges):
        if hi > lo:
            part = [np.ascontiguousarray(inp[k][:, lo:hi]) for k in GDN_KEYS]
            ro = cref.gated_deltanet2(*part, None, scale=s.scale, use_qk_l2norm=s.l2norm, dtype=np.float64)
            check(f"gdn2_packed_gaps/{case}/{gdn2_path}/seq{n}", o[:, lo:hi], ro, TOL_GDN2)


@pytest.mark.parametrize("case", sorted(GAP_CASES))
def test_m3_packed_uncovered_rows_are_zero(case, m3_path):
    import torch
    cu, T = GAP_CASES[case]
    s = W.Mamba3SisoShape(1, T, 2, 16, 32, has_z=True)
    inp = W.mamba3_siso_inputs(s, seed=52)
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda")
    call = mamba3_siso_fn(*(to_dev(inp[k]) for k in M3_KEYS), cu_seqlens=cu_t, prepare=True)
    call.out.fill_(float("nan"))
    y = call().cpu().numpy()
    cov, ranges = _covered(cu, T)
    assert np.all(y[:, ~cov] == 0.0)
    for n, (lo, hi) in enumerate(ranges):
        if hi > lo:
            part = {}
            for k in M3_KEYS:
                x = inp[k]
                if x is None or k in ("Q_bias", "K_bias", "D"):
                    part[k] = x
                elif k in ("ADT", "DT", "Trap"):
                    part[k] = np.ascontiguousarray(x[:, :, lo:hi])
                else:
                    part[k] = np.ascontiguousarray(x[:, lo:hi])
            ry = cref.mamba3_siso(*(part[k] for k in M3_KEYS), dtype=np.float64)
            check(f"m3_packed_gaps/{case}/{m3_path}/seq{n}", y[:, lo:hi], ry, TOL_M3)


@pytest.mark.parametrize("dk,dv", [(64, 40), (128, 65), (256, 20)])
def test_gdn2_packed_two_column_tiles(dk, dv, override):
    """Packed sequences through the two-tile recurrence (gdn2_ct = 2)."""
    override("gdn2_ct", 2)
    gdn2_packed_check([37, 0, 1, 16, 50, 700], 2, dk, dv, True, "chunk", 13, f"gdn2_packed_ct2/{dk}x{dv}")
