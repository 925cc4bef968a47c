"""GatedDeltaNet2Fn on the GPU vs the fp64 oracle (C restatement), through
the C ABI.  Covers the reference's dispatch boundaries: key dimensions on
both sides of 256 (VGPR-state and LDS-state paths), partial waves (value
dims that are not multiples of the column tiling), initial states, Q/K
normalisation on and off, several batches, token counts around the
1024-token preparation chunk, and overlapping calls on one device.

Three device paths: the chunked fp32-MFMA kernel (dk <= 512, the default
there), the token-sequential register kernel (dk <= 512; forced with
the gdn2_path override, and taken by packed sequences) and the LDS-state kernel
(dk > 512).  The
parity cases run on both paths where both apply; the chunked path's
pairwise fallback (forced with the gdn2_pairwise override, or taken by chunks with
extreme decays) has its own cases."""

import numpy as np
import pytest

from oracle import cref
from parity import TOL_GDN2, check, to_dev
import xmetai_onnx_plugins as xp
from xmetai_onnx_plugins import TorchAllocator, gated_deltanet2_fn, workloads as W

pytestmark = pytest.mark.gpu

KEYS = ("q", "k", "v", "g", "beta", "w", "initial_state")


def run_gpu(inp, s, **kw):
    import torch
    y = gated_deltanet2_fn(*(to_dev(inp[k]) for k in KEYS), scale=s.scale, use_qk_l2norm_in_kernel=s.l2norm, **kw)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def run_ref(inp, s, dtype=np.float64):
    return cref.gated_deltanet2(*(inp[k] for k in KEYS), scale=s.scale, use_qk_l2norm=s.l2norm, dtype=dtype)


S = W.GatedDeltaNet2Shape
CASES = {
    "k1_v1": S(1, 9, 2, 1, 1),
    "t1_single_token": S(2, 1, 3, 64, 32),
    "t3_shorter_than_block": S(1, 3, 2, 128, 40, per_key_gates=True),
    "t9_big_grid_one_block_plus_one": S(8, 9, 16, 64, 64),
    "k16_v16": S(2, 33, 3, 16, 16),
    "k17_v15_partial": S(2, 20, 2, 17, 15),
    "k32_v33_nos0": S(1, 40, 2, 32, 33, initial_state=False),
    "k64_v64_perkey": S(2, 50, 2, 64, 64, per_key_gates=True),
    "k80_v24_three_waves": S(2, 45, 2, 80, 24),
    "k96_t2100_three_waves_window_carry": S(1, 2100, 1, 96, 16, per_key_gates=True),
    "k100_v48": S(1, 31, 3, 100, 48),
    "k128_v128_nol2": S(1, 24, 2, 128, 128, l2norm=False),
    "k128_v65_partial_wave": S(2, 64, 4, 128, 65),
    "k200_v40": S(1, 17, 2, 200, 40),
    "k256_v256": S(1, 48, 2, 256, 256),
    "k257_two_rows": S(1, 21, 2, 257, 20),
    "k320_v64": S(2, 40, 2, 320, 64),
    "k352_v20_chunk12": S(1, 37, 2, 352, 20),
    "k384_v16": S(1, 33, 1, 384, 16, per_key_gates=True),
    # 128 column-tile workgroups: 352 keys take 6 key tiles per wave x 4 waves
    "k352_v256_h8_six_tiles": S(1, 40, 8, 352, 256, per_key_gates=True),
    "k385_v16": S(1, 19, 1, 385, 16),
    "k448_v40": S(2, 35, 1, 448, 40),
    "k512_v7_perkey": S(1, 12, 1, 512, 7, per_key_gates=True),
    "k513_lds_path": S(1, 21, 2, 513, 20),
    "k600_v33_lds_path": S(2, 40, 2, 600, 33),
    "k1024_lds_path_perkey": S(1, 12, 1, 1024, 7, per_key_gates=True),
    "t1023": S(1, 1023, 2, 32, 16),
    "t1024": S(1, 1024, 2, 32, 16),
    "t1025_chunk_carry": S(1, 1025, 2, 32, 16),
    "t2100_two_carries": S(2, 2100, 1, 64, 32, per_key_gates=True),
    "t2100_k320_window_carry": S(1, 2100, 1, 320, 16),
    "t2060_k512_window_carry_perkey": S(1, 2060, 1, 512, 8, per_key_gates=True),
    "t1500_lds_carry": S(1, 1500, 1, 600, 16),
    # above 2048 keys the state tile lives in scratch (any head_k, as the
    # reference's generic kernel): 1100 tokens cross one preparation-chunk carry
    "k2049_v20_tile_store": S(1, 40, 2, 2049, 20),
    "k4096_v64_t1100_carry": S(1, 1100, 1, 4096, 64),
    "k4096_v64_t1100_carry_nos0": S(1, 1100, 1, 4096, 64, initial_state=False),
    "k3000_v33_perkey": S(2, 30, 1, 3000, 33, per_key_gates=True),
}


@pytest.mark.parametrize("path", ["default", "seq"])
@pytest.mark.parametrize("name", sorted(CASES))
def test_gdn2_parity(name, path, override):
    s = CASES[name]
    if path == "seq":
        if s.dk > 512:
            pytest.skip("dk > 512 has one path")
        override("gdn2_path", 1)
    inp = W.gated_deltanet2_inputs(s, seed=0)
    # without the L2 norm the state explodes: gated against the fp32-order oracle's own error
    ref32 = None if s.l2norm else run_ref(inp, s, np.float32)
    check(f"gated_deltanet2/{name}/{path}", run_gpu(inp, s), run_ref(inp, s), TOL_GDN2, ref32=ref32)


WINDOW_CASES = ["k96_t2100_three_waves_window_carry", "t2100_two_carries", "t2100_k320_window_carry",
                "t2060_k512_window_carry_perkey"]


@pytest.mark.parametrize("name", WINDOW_CASES)
def test_gdn2_windows_of_128_chunks(name, override):
    """The chunked path stepped in 128-chunk windows (gdn2_windowed; the
    default sizes windows to 128 MiB of blocks, one window at these shapes):
    the state crosses windows through the carry."""
    import xmetai_onnx_plugins as xp
    s = CASES[name]
    override("gdn2_windowed", 1)
    inp = W.gated_deltanet2_inputs(s, seed=0)
    got = run_gpu(inp, s)
    assert any(k.startswith("Gdn2ChunkPrepKernel x") for k in xp.last_launches()), xp.last_launches()
    check(f"gated_deltanet2/{name}/windows128", got, run_ref(inp, s), TOL_GDN2)


@pytest.mark.parametrize("shape", [(1, 37, 2, 64, 40), (2, 50, 2, 128, 33), (1, 20, 1, 256, 16), (1, 9, 2, 5, 3)])
def test_gdn2_chunk_pairwise_fallback(shape, override):
    """The chunked path with every chunk on the pairwise decay products."""
    s = S(*shape, per_key_gates=True)
    inp = W.gated_deltanet2_inputs(s, seed=9)
    override("gdn2_pairwise", 1)
    check("gated_deltanet2/pairwise_" + "_".join(map(str, shape)), run_gpu(inp, s), run_ref(inp, s), TOL_GDN2)


@pytest.mark.parametrize("g", [-30.0, -200.0, 3.0])
def test_gdn2_chunk_extreme_decay(g):
    """Chunks whose cumulative decay leaves [2^-60, 2^60] (a hard reset of some
    keys, or growth) take the pairwise products; the others the fast form."""
    s = S(2, 90, 2, 64, 24, per_key_gates=True)
    inp = W.gated_deltanet2_inputs(s, seed=10)
    inp["g"] = inp["g"].copy()
    inp["g"][:, 20] = g                    # every key of token 20
    inp["g"][1, 47, :, :9] = g             # some keys of one token
    if g > 0:
        inp["g"][:, 60:80] = g             # growth: e^48 over the chunk of tokens 64-79
    check(f"gated_deltanet2/extreme_{g}", run_gpu(inp, s), run_ref(inp, s), TOL_GDN2,
          ref32=run_ref(inp, s, np.float32))


@pytest.mark.parametrize("shape", [(8, 40, 32, 64, 32), (4, 30, 16, 64, 96), (2, 20, 16, 400, 128),
                                   (2, 70, 2, 128, 96), (1, 19, 2, 256, 200)])
def test_gdn2_workgroup_shapes(shape):
    """The automatic choice: 1, 2 or 4 rows of 16 lanes per value column (2
    rows for dk = 400), 8- or 4-wave workgroups, partial column blocks and
    token counts that end inside a block."""
    s = S(*shape)
    inp = W.gated_deltanet2_inputs(s, seed=3)
    check("gated_deltanet2/wg_" + "_".join(map(str, shape)), run_gpu(inp, s), run_ref(inp, s), TOL_GDN2)


@pytest.mark.parametrize("rows", [1, 2, 4])
@pytest.mark.parametrize("shape", [(2, 37, 3, 64, 40), (1, 45, 2, 200, 24)])
def test_gdn2_rows_per_column_agree(rows, shape, override):
    """Every column layout of the sequential kernel (forced through the
    gdn2_rows override where the keys fit) matches the oracle on the same inputs."""
    s = S(*shape)
    inp = W.gated_deltanet2_inputs(s, seed=7)
    override("gdn2_path", 1)
    override("gdn2_rows", rows)
    check(f"gated_deltanet2/rows{rows}_" + "_".join(map(str, shape)), run_gpu(inp, s), run_ref(inp, s), TOL_GDN2)


def test_gdn2_torch_allocator_and_overlapping_streams():
    """Two calls in flight on two streams, one on the fused path (no scratch)
    and one on the large-key path with scratch from torch's caching allocator
    (1100 tokens: two preparation chunks): each matches its own oracle result."""
    import torch
    s1, s2 = S(1, 1100, 2, 600, 24), S(1, 700, 3, 128, 40)
    i1, i2 = W.gated_deltanet2_inputs(s1, seed=5), W.gated_deltanet2_inputs(s2, seed=6)
    d1 = [to_dev(i1[k]) for k in KEYS]
    d2 = [to_dev(i2[k]) for k in KEYS]
    st1, st2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    a1, a2 = TorchAllocator(stream=st1), TorchAllocator(stream=st2)
    with torch.cuda.stream(st1):
        y1 = gated_deltanet2_fn(*d1, scale=s1.scale, allocator=a1)
    with torch.cuda.stream(st2):
        y2 = gated_deltanet2_fn(*d2, scale=s2.scale, allocator=a2)
    torch.cuda.synchronize()
    assert a1.live == 0 and a2.live == 0
    check("gated_deltanet2/overlap_1", y1.cpu().numpy(), run_ref(i1, s1), TOL_GDN2)
    check("gated_deltanet2/overlap_2", y2.cpu().numpy(), run_ref(i2, s2), TOL_GDN2)


def _head_subset(inp, b, hs):
    sub = {}
    for k in ("q", "k", "v", "g", "beta", "w"):
        sub[k] = np.ascontiguousarray(inp[k][b:b + 1, :, hs])
    sub["initial_state"] = None if inp["initial_state"] is None else np.ascontiguousarray(inp["initial_state"][b:b + 1, hs])
    return sub


@pytest.mark.parametrize("name", ["gated_deltanet2_b4_t4096_h16_k128_v128", "gated_deltanet2_b1_t16384_h8_k256_v256",
                                  "gated_deltanet2_b2_t2048_h4_k320_v64", "gated_deltanet2_b4_t4096_h16_k128_v65"])
def test_gdn2_benchmark_shapes(name):
    """Benchmark shapes: heads are independent, so a subset of (batch, head)
    pairs is checked against the oracle over the full sequence."""
    import torch
    s = W.NAMED[name]
    inp = W.gated_deltanet2_inputs(s, seed=0)
    y = run_gpu(inp, s)
    b, hs = s.batch - 1, [0, s.nheads - 1] if s.nheads > 1 else [0]
    sub = _head_subset(inp, b, hs)
    ref = cref.gated_deltanet2(*(sub[k] for k in KEYS), scale=s.scale, use_qk_l2norm=s.l2norm, dtype=np.float64)
    check(f"gated_deltanet2/{name}_heads", y[b:b + 1, :, hs], ref, TOL_GDN2)
    assert np.isfinite(y).all()


# Sequence split (gdn2_split override 2: up to four segments wherever the
# sequence has two or more chunks): segments after the first run from a zero
# state beside identity columns, and their outputs are corrected afterwards.
SPLIT_CASES = {
    "t50_k100_v48_one_chunk_segments": S(1, 50, 3, 100, 48),
    "t300_k128_v65": S(1, 300, 2, 128, 65),
    "t600_k64_v32": S(1, 600, 2, 64, 32),
    "t1000_k17_v15_nos0": S(2, 1000, 1, 17, 15, initial_state=False),
    "t700_k320_v20_perkey": S(1, 700, 1, 320, 20, per_key_gates=True),
    "t520_k512_v7": S(1, 520, 1, 512, 7),
    "t1025_k256_v256": S(1, 1025, 1, 256, 256),
    "t40_k128_v128_nol2": S(1, 40, 1, 128, 128, l2norm=False),   # the state grows ~60x a token
    "t32_k96_v40_two_segments": S(2, 32, 2, 96, 40),   # two segments: no combine step
}


@pytest.mark.parametrize("name", sorted(SPLIT_CASES))
def test_gdn2_sequence_split(name, override):
    s = SPLIT_CASES[name]
    inp = W.gated_deltanet2_inputs(s, seed=4)
    override("gdn2_split", 2)
    got = run_gpu(inp, s)
    assert any(k.startswith("Gdn2ChunkSplitKernel") for k in xp.last_launches()), xp.last_launches()
    ref32 = None if s.l2norm else run_ref(inp, s, np.float32)
    check(f"gated_deltanet2/split_{name}", got, run_ref(inp, s), TOL_GDN2, ref32=ref32)


# Two unequal segments, the second at two column tiles per workgroup
# (gdn2_split override 3; key tilings with a two-tile kernel, up to 256 keys).
# Odd value-tile counts leave the last value pair half empty, odd key-tile
# counts the last identity pair (its second tile past the padded keys stores
# nothing).
SPLIT2_CASES = {
    "t50_k100_v48": S(1, 50, 3, 100, 48),
    "t300_k128_v65_odd_value_tiles": S(1, 300, 2, 128, 65),
    "t600_k64_v32": S(1, 600, 2, 64, 32),
    "t1000_k40_v15_odd_key_tiles_nos0": S(2, 1000, 1, 40, 15, initial_state=False),
    "t700_k160_v48_perkey": S(1, 700, 1, 160, 48, per_key_gates=True),
    "t1025_k256_v256": S(1, 1025, 1, 256, 256),
    "t40_k128_v128_nol2": S(1, 40, 1, 128, 128, l2norm=False),
    "t17_k33_v17_two_chunks": S(1, 17, 2, 33, 17),
}


@pytest.mark.parametrize("name", sorted(SPLIT2_CASES))
def test_gdn2_two_tile_split(name, override):
    s = SPLIT2_CASES[name]
    inp = W.gated_deltanet2_inputs(s, seed=12)
    override("gdn2_split", 3)
    got = run_gpu(inp, s)
    assert any(k.startswith("Gdn2ChunkSplit2Kernel") for k in xp.last_launches()), xp.last_launches()
    ref32 = None if s.l2norm else run_ref(inp, s, np.float32)
    check(f"gated_deltanet2/split2_{name}", got, run_ref(inp, s), TOL_GDN2, ref32=ref32)


def test_gdn2_two_tile_split_selected_for_wide_heads():
    """1 x 8 heads at 256 x 256 (128 value-tile workgroups, too many value and
    key tiles for a second segment at one tile each) takes the two-tile split
    by itself; the first and last heads are checked over the whole sequence."""
    s = S(1, 2048, 8, 256, 256, initial_state=False)
    inp = W.gated_deltanet2_inputs(s, seed=13)
    y = run_gpu(inp, s)
    launched = xp.last_launches()
    assert any(k.startswith("Gdn2ChunkSplit2Kernel") for k in launched), launched
    assert not any(k.startswith("Gdn2SplitCombineKernel") for k in launched), launched
    sub = _head_subset(inp, 0, [0, 7])
    ref = cref.gated_deltanet2(*(sub[k] for k in KEYS), scale=s.scale, use_qk_l2norm=s.l2norm, dtype=np.float64)
    check("gated_deltanet2/split2_auto_heads", y[:, :, [0, 7]], ref, TOL_GDN2)


def test_gdn2_two_segment_split_without_combine():
    """Wide keys over few value columns split into two segments by default;
    with no final state requested segment 0's final state is segment 1's start
    and no combine kernel runs.  With the final state the combine forms it."""
    import torch
    s = S(2, 1024, 4, 320, 64)
    inp = W.gated_deltanet2_inputs(s, seed=6)
    got = run_gpu(inp, s)
    launched = xp.last_launches()
    assert any(k.startswith("Gdn2ChunkSplitKernel") for k in launched), launched
    assert not any(k.startswith("Gdn2SplitCombineKernel") for k in launched), launched
    check("gated_deltanet2/split_two_segments", got, run_ref(inp, s), TOL_GDN2)
    y, st = gated_deltanet2_fn(*(to_dev(inp[k]) for k in KEYS), scale=s.scale, output_final_state=True)
    torch.cuda.synchronize()
    assert any(k.startswith("Gdn2SplitCombineKernel") for k in xp.last_launches()), xp.last_launches()
    np.testing.assert_array_equal(y.cpu().numpy(), got)


def test_gdn2_sequence_split_selected_for_few_workgroups(override):
    """A call with few column-tile workgroups and 64+ chunks splits its
    sequence by itself; gdn2_split = 1 keeps one recurrence over the windows."""
    s = S(1, 1024, 2, 64, 32)
    inp = W.gated_deltanet2_inputs(s, seed=5)
    got = run_gpu(inp, s)
    assert any(k.startswith("Gdn2ChunkSplitKernel") for k in xp.last_launches()), xp.last_launches()
    override("gdn2_split", 1)
    whole = run_gpu(inp, s)
    assert not any(k.startswith("Gdn2ChunkSplitKernel") for k in xp.last_launches()), xp.last_launches()
    ref = run_ref(inp, s)
    check("gated_deltanet2/split_auto", got, ref, TOL_GDN2)
    check("gated_deltanet2/split_off", whole, ref, TOL_GDN2)


def test_gdn2_column_independence_bitwise():
    """Column j of the output depends only on column j of v, w and S0: a
    dv=65 run equals the first 65 columns of a dv=128 run, bit for bit."""
    import torch
    s128 = S(1, 300, 2, 128, 128)
    inp = W.gated_deltanet2_inputs(s128, seed=9)
    y128 = run_gpu(inp, s128)
    sub = dict(inp)
    for k in ("v", "w"):
        sub[k] = np.ascontiguousarray(inp[k][..., :65])
    sub["initial_state"] = np.ascontiguousarray(inp["initial_state"][..., :65])
    y65 = run_gpu(sub, S(1, 300, 2, 128, 65))
    np.testing.assert_array_equal(y65, y128[..., :65])


def test_gdn2_split_scratch_refused_falls_back_to_windows():
    """An allocator that refuses the sequence split's scratch (every chunk's
    blocks at once) still gets a successful call: the operator asks again
    for the windowed plan's bytes, which it grants, and the result matches
    the oracle."""
    import torch
    s = S(1, 4096, 2, 128, 64)   # few heads, 256 chunks: the split is the default plan
    inp = W.gated_deltanet2_inputs(s, seed=17)
    split_bytes = xp.validate("gated_deltanet2", [inp[k].shape if inp[k] is not None else None for k in KEYS])[1]
    base = TorchAllocator()
    asked = []

    def refusing(ctx, nbytes):
        asked.append(int(nbytes))
        return None if nbytes >= split_bytes else base._alloc_cb(ctx, nbytes)

    from xmetai_onnx_plugins import _capi
    alloc = TorchAllocator()
    alloc._alloc_cb = _capi.ALLOC_FN(refusing)
    alloc.struct = _capi.XmAllocator(None, alloc._alloc_cb, base._free_cb)
    y = gated_deltanet2_fn(*(to_dev(inp[k]) for k in KEYS), scale=s.scale, use_qk_l2norm_in_kernel=s.l2norm,
                           allocator=alloc)
    torch.cuda.synchronize()
    launched = xp.last_launches()
    assert len(asked) == 2 and asked[0] == split_bytes and asked[1] < split_bytes, asked
    assert not any(k.startswith("Gdn2ChunkSplitKernel") for k in launched), launched
    assert any(k.startswith("Gdn2ChunkRecurKernel") for k in launched), launched
    check("gated_deltanet2/split_refused_windows", y.cpu().numpy(), run_ref(inp, s), TOL_GDN2)


# Two value-column tiles per recurrence workgroup (gdn2_ct = 2; built for 33 to
# 256 keys): the key tiles' operands serve 32 columns, a workgroup's last tile
# may be past dv (ragged dv), and the state of both tiles crosses windows.
CT2_CASES = [n for n in sorted(CASES) if 32 < CASES[n].dk <= 256]


def _ran_two_tiles():
    return any(k.startswith("Gdn2ChunkRecurKernel<") and k.split("<")[1].split(",")[2] == "2"
               for k in xp.last_launches())


@pytest.mark.parametrize("name", CT2_CASES)
def test_gdn2_parity_two_column_tiles(name, override):
    s = CASES[name]
    override("gdn2_ct", 2)
    override("gdn2_split", 1)   # the recurrence kernel itself, not the sequence split
    inp = W.gated_deltanet2_inputs(s, seed=0)
    got = run_gpu(inp, s)
    assert _ran_two_tiles(), xp.last_launches()
    ref32 = None if s.l2norm else run_ref(inp, s, np.float32)
    check(f"gated_deltanet2/{name}/ct2", got, run_ref(inp, s), TOL_GDN2, ref32=ref32)


@pytest.mark.parametrize("shape", [(1, 2100, 2, 96, 40, True), (2, 4100, 1, 64, 24, False), (1, 2100, 1, 192, 33, True)])
def test_gdn2_two_column_tiles_window_carry(shape, override):
    """128-chunk windows (gdn2_windowed): both column tiles' states carried."""
    b, t, h, k, v, perkey = shape
    s = S(b, t, h, k, v, per_key_gates=perkey)
    override("gdn2_ct", 2)
    override("gdn2_windowed", 1)
    inp = W.gated_deltanet2_inputs(s, seed=11)
    got = run_gpu(inp, s)
    assert _ran_two_tiles(), xp.last_launches()
    check(f"gated_deltanet2/ct2_windows_{b}_{t}_{h}_{k}_{v}", got, run_ref(inp, s), TOL_GDN2)


@pytest.mark.parametrize("shape, two", [((4, 40, 16, 128, 65), True),    # 320 one-tile workgroups
                                         ((4, 40, 12, 128, 128), True),   # 384
                                         ((2, 40, 16, 128, 128), False),  # 256: one per CU already
                                         ((4, 40, 16, 64, 64), False)])   # 256
def test_gdn2_two_column_tiles_by_default_above_one_workgroup_per_cu(shape, two):
    """Without the override the recurrence takes two column tiles exactly where
    one tile per workgroup would launch more workgroups than the 256 CUs."""
    s = S(*shape)
    inp = W.gated_deltanet2_inputs(s, seed=13)
    got = run_gpu(inp, s)
    assert _ran_two_tiles() == two, xp.last_launches()
    check("gated_deltanet2/ct_default_" + "_".join(map(str, shape)), got, run_ref(inp, s), TOL_GDN2)


def test_gdn2_two_column_tiles_equal_one_bitwise(override):
    """Columns are independent and both layouts sum in the same order: two
    tiles per workgroup give the one-tile results bit for bit (dv = 65: the
    third workgroup's second tile is past dv)."""
    s = S(2, 300, 3, 128, 65)
    inp = W.gated_deltanet2_inputs(s, seed=12)
    override("gdn2_split", 1)
    override("gdn2_ct", 1)
    one = run_gpu(inp, s)
    override("gdn2_ct", 2)
    two = run_gpu(inp, s)
    assert _ran_two_tiles(), xp.last_launches()
    np.testing.assert_array_equal(two, one)
