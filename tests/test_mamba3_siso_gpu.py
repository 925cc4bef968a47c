"""Mamba3SisoFn on the GPU vs the fp64 oracle (C restatement), through the
C ABI, for both kernels (the chunked fp32-MFMA kernel and, with
the m3_path override, the token-by-token one).  Covers headdim_qk padding (N not a
multiple of the key tiling), headdim_qk above 512 (key-block launches), partial angle sets (A < N/2), grouped Q/K heads,
the optional D and Z inputs, sequence lengths around the 16-token chunk and
block, the 32-row workgroups, decay patterns, and the benchmark shape on a
subset of heads."""

import numpy as np
import pytest

from oracle import cref
from parity import TOL_GPU, TOL_M3, check, to_dev
from xmetai_onnx_plugins import mamba3_siso_fn, workloads as W

pytestmark = pytest.mark.gpu

KEYS = ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")


def run_gpu(inp):
    import torch
    y = mamba3_siso_fn(*(to_dev(inp[k]) for k in KEYS))
    torch.cuda.synchronize()
    return y.cpu().numpy()


def run_ref(inp, dtype=np.float64):
    return cref.mamba3_siso(*(inp[k] for k in KEYS), dtype=dtype)


M = W.Mamba3SisoShape
CASES = {
    "t1": M(2, 1, 2, 8, 16),
    "t2_z": M(1, 2, 2, 8, 16, has_z=True),
    "n2_a1": M(1, 20, 2, 5, 2),
    "n8_p7": M(2, 17, 3, 7, 8),
    "n16_t16": M(1, 16, 2, 16, 16),
    "n64_p33_hq1": M(1, 33, 4, 33, 64, nheads_qk=1),
    "n128_a7_partial_angles": M(1, 40, 2, 64, 128, angles=7),
    "n128_p64_z_no_d": M(1, 50, 2, 64, 128, has_d=False, has_z=True),
    "n130_padded": M(1, 25, 2, 20, 130),
    "n192": M(1, 19, 2, 16, 192),
    "n256": M(1, 21, 2, 24, 256),
    # above 256 keys the token-by-token kernel runs on either setting (24 and
    # 32 keys per lane, each token's q / k read from LDS)
    "n384_p64_z": M(1, 40, 2, 64, 384, has_z=True),
    "n512_p64_z": M(2, 37, 2, 64, 512, has_z=True),
    "n512_a50_t70": M(1, 70, 1, 40, 512, angles=50),
    # above 512 keys: one launch per 512-key block, each adding its part of y
    # (angles inside the first block, crossing into the second, a partial last
    # block, a shared Q/K head, two row blocks, Z applied by the last launch)
    "n1024_p16_z_a100": M(1, 45, 2, 16, 1024, has_z=True, angles=100),
    "n1100_p24_a300_hq1": M(1, 33, 2, 24, 1100, nheads_qk=1, angles=300),
    "n640_p40_z": M(2, 30, 2, 40, 640, has_z=True),
    "p65_rowblocks": M(2, 35, 2, 65, 32),
    "t100_hq2": M(2, 100, 4, 16, 32, nheads_qk=2),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_mamba3_parity(name, m3_path):
    s = CASES[name]
    inp = W.mamba3_siso_inputs(s, seed=0)
    check(f"mamba3_siso/{name}", run_gpu(inp), run_ref(inp), TOL_M3)


@pytest.mark.parametrize("shape", [(2, 33, 2, 65, 64), (1, 17, 2, 100, 256), (1, 64, 2, 32, 128),
                                   (1, 47, 3, 97, 192), (2, 31, 2, 3, 32)])
def test_mamba3_row_blocks_and_ragged_token_blocks(shape, m3_path):
    """Several 32-row workgroups per head with a partial last one, token counts
    that end inside a 16-token chunk or a 32-token block, Z present."""
    s = M(*shape, has_z=True)
    inp = W.mamba3_siso_inputs(s, seed=4)
    check("mamba3_siso/rows_" + "_".join(map(str, shape)), run_gpu(inp), run_ref(inp), TOL_M3)


@pytest.mark.parametrize("pattern", ["mild", "mixed", "steep", "growth"])
def test_mamba3_decay_patterns(pattern, m3_path):
    """Decay patterns: mild, alternating mild / steep 32-token stretches,
    underflowing decays (-100 per token every 7th), and growth (+0.9 / -0.5).
    The chunked kernel forms e^{cum_t - cum_s} per pair, so a steep stretch
    underflows to zero exactly where the token-by-token product does."""
    s = M(2, 150, 2, 24, 64, has_z=pattern == "mixed")
    inp = W.mamba3_siso_inputs(s, seed=11)
    t = np.arange(s.seqlen)
    if pattern == "mild":
        adt = np.full(s.seqlen, -0.3)
    elif pattern == "mixed":
        adt = np.where((t // 32) % 2 == 0, -0.2, -5.0)          # alternating scaled / unscaled blocks
    elif pattern == "steep":
        adt = np.where(t % 7 == 3, -100.0, -2.0)                # underflowing decays
    else:
        adt = np.where(t % 2 == 0, 0.9, -0.5)                   # growth within the bound
    inp["ADT"] = np.broadcast_to(adt.astype(np.float32), inp["ADT"].shape).copy()
    check(f"mamba3_siso/decay_{pattern}", run_gpu(inp), run_ref(inp), TOL_M3, ref32=run_ref(inp, np.float32))


def test_mamba3_long_angle_accumulation(m3_path):
    """4096 steps with large angle increments: the wrapped angle state must not
    drift from the fp64 oracle (the device accumulates it in fp64)."""
    s = M(1, 4096, 1, 8, 16)
    inp = W.mamba3_siso_inputs(s, seed=5)
    inp["DT"] = np.full_like(inp["DT"], 2.0)
    inp["ADT"] = np.full_like(inp["ADT"], -0.05)
    check("mamba3_siso/long_angles", run_gpu(inp), run_ref(inp), TOL_M3, ref32=run_ref(inp, np.float32))


def test_mamba3_benchmark_shape_heads(m3_path):
    """Benchmark shape 4 x 4096 x 32 heads, P=64, N=128: (b,h) pairs are
    independent; a subset is checked against the oracle over all 4096 tokens."""
    s = W.M3_MAIN
    inp = W.mamba3_siso_inputs(s, seed=0)
    y = run_gpu(inp)
    b, hs = s.batch - 1, [0, 17, s.nheads - 1]
    sub = {}
    for k in ("Q", "K", "V", "Angles"):
        sub[k] = np.ascontiguousarray(inp[k][b:b + 1, :, hs])
    for k in ("ADT", "DT", "Trap"):
        sub[k] = np.ascontiguousarray(inp[k][b:b + 1, hs])
    for k in ("Q_bias", "K_bias"):
        sub[k] = np.ascontiguousarray(inp[k][hs])
    sub["D"] = np.ascontiguousarray(inp["D"][hs])
    sub["Z"] = None
    check("mamba3_siso/b4_t4096_h32_p64_n128_heads", y[b:b + 1, :, hs], run_ref(sub), TOL_M3)
    assert np.isfinite(y).all()


def test_mamba3_long_sequence(m3_path):
    """65536 tokens (4096 chunks): chunk offsets far into the buffers and the
    angle carry over many chunks, against the oracle."""
    s = M(1, 65536, 1, 16, 16, angles=8)
    inp = W.mamba3_siso_inputs(s, seed=21)
    check("mamba3_siso/t65536", run_gpu(inp), run_ref(inp), TOL_M3)


def test_mamba3_path_switch_selects_the_other_kernel(override):
    """The m3_path override runs the token-by-token kernel: its summation order
    differs from the chunked kernel's, so the two outputs are close but not
    bit-identical (both kernels are then exercised by the tests above)."""
    s = M(1, 64, 2, 32, 64)
    inp = W.mamba3_siso_inputs(s, seed=22)
    import xmetai_onnx_plugins as xp
    override("m3_path", 0)
    chunked = run_gpu(inp)
    assert xp.last_launches() == ["Mamba3ChunkKernel<1,4,4,0>"]
    override("m3_path", 1)
    sequential = run_gpu(inp)
    assert xp.last_launches() == ["Mamba3FwdKernel<4>"]
    assert not np.array_equal(chunked, sequential)
    check("mamba3_siso/chunked_vs_seq", chunked, sequential, TOL_GPU)


def test_mamba3_token_rows_past_2gib(m3_path):
    """1 x 65536 tokens x 64 heads, P = 128, N = 16 with Z: the V, Z and output
    token rows of the sequence span 2 GiB each, past a buffer descriptor's
    32-bit range, so the chunked kernel reads and writes through per-chunk
    descriptors (LONG).  Inputs are drawn on the device with the benchmark's
    distributions; heads 0 and 41 over all 65536 tokens against the oracle."""
    import math
    import torch
    import xmetai_onnx_plugins as xp
    from xmetai_onnx_plugins import mamba3_siso_fn
    B, T, H, P, N, A = 1, 65536, 64, 128, 16, 8
    g = torch.Generator(device="cuda")
    g.manual_seed(31)
    rn = lambda *shape: torch.randn(shape, generator=g, device="cuda")
    ru = lambda *shape: torch.rand(shape, generator=g, device="cuda")
    V = rn(B, T, H, P)
    DT = torch.nn.functional.softplus(rn(B, H, T) + (-4.0 + 2.0 * ru(H))[None, :, None])
    ADT = -torch.exp(ru(H) * math.log(16.0))[None, :, None] * DT
    Q, K = rn(B, T, H, N) / math.sqrt(N), rn(B, T, H, N) / math.sqrt(N)
    Trap, Angles, D = ru(B, H, T), ru(B, T, H, A), rn(H)
    Qb, Kb = rn(H, N) / math.sqrt(N), rn(H, N) / math.sqrt(N)
    Z = rn(B, T, H, P)
    y = mamba3_siso_fn(Q, K, V, ADT, DT, Trap, Qb, Kb, Angles, D, Z)
    torch.cuda.synchronize()
    if m3_path == "chunk":
        assert xp.last_launches() == ["Mamba3ChunkKernel<1,4,4,1>"], xp.last_launches()
    hs = [0, 41]
    host = lambda x: np.ascontiguousarray(x.cpu().numpy())
    sub = dict(Q=host(Q[:, :, hs]), K=host(K[:, :, hs]), V=host(V[:, :, hs]), ADT=host(ADT[:, hs]),
               DT=host(DT[:, hs]), Trap=host(Trap[:, hs]), Q_bias=host(Qb[hs]), K_bias=host(Kb[hs]),
               Angles=host(Angles[:, :, hs]), D=host(D[hs]), Z=host(Z[:, :, hs]))
    got = host(y[:, :, hs])
    del V, Z, y
    torch.cuda.empty_cache()
    check(f"mamba3_siso/t65536_h64_p128_rows_past_2gib/{m3_path}", got, run_ref(sub), TOL_M3)
