"""xm_gated_deltanet2_forward_noalloc: GatedDeltaNet2Fn with its scratch in a
fixed 64 MiB device array instead of an allocator (for callers that cannot
allocate), called through the C ABI.  Its outputs must equal those of
xm_gated_deltanet2_forward on the same inputs, on consecutive calls that
reuse the array (the second smaller than the first), on the chunked path
with windows shrunk to fit the array, on the sequence-split path, and on the
dk > 512 paths; where the allocating call splits the sequence into more
scratch than the array holds, the two agree within the device-path
tolerance."""

import ctypes

import numpy as np
import pytest

import xmetai_onnx_plugins as xp
from xmetai_onnx_plugins import _capi, workloads as W
from parity import TOL_GPU, check, to_dev

S = W.GatedDeltaNet2Shape
KEYS = ("q", "k", "v", "g", "beta", "w", "initial_state")


def _entry():
    return xp.lib().xm_gated_deltanet2_forward_noalloc   # argument types declared in _capi


def _call_noalloc(descs, s, out_ptr, stream_ptr, **extra):
    arr = (_capi.XmTensor * len(descs))(*descs)
    attrs = xp._attrs("gated_deltanet2", scale=s.scale, use_qk_l2norm_in_kernel=int(s.l2norm), **extra)
    err = ctypes.create_string_buffer(512)
    st = _entry()(arr, len(descs), ctypes.byref(attrs), out_ptr, stream_ptr, err, len(err))
    return st, err.value.decode()


def run_both(s, seed):
    """(noalloc output, allocating entry point's output) on the same device inputs."""
    import torch
    inp = W.gated_deltanet2_inputs(s, seed=seed)
    d = {k: to_dev(inp[k]) for k in KEYS}
    ref = xp.gated_deltanet2_fn(*(d[k] for k in KEYS), scale=s.scale, use_qk_l2norm_in_kernel=int(s.l2norm))
    out = torch.full_like(ref, float("nan"))
    stream = torch.cuda.current_stream()
    st, msg = _call_noalloc([xp._desc_from_tensor(d[k]) for k in KEYS], s, out.data_ptr(), stream.cuda_stream)
    assert st == xp.XM_OK, msg
    launched = xp.last_launches()
    torch.cuda.synchronize()
    return out.cpu().numpy(), ref.cpu().numpy(), launched


@pytest.mark.gpu
def test_noalloc_equals_the_allocating_entry_point_on_consecutive_calls():
    # 1: 64 heads x 2100 tokens at 128 x 64 needs 223 MB of prepared blocks with
    #    128-chunk windows; in 64 MiB the windows shrink (carry between them)
    got, want, launched = run_both(S(4, 2100, 16, 128, 64), seed=1)
    np.testing.assert_array_equal(got, want)
    assert any(k.startswith("Gdn2ChunkRecurKernel") for k in launched), launched
    # 2: a smaller call right after, on the same array
    got, want, _ = run_both(S(1, 300, 2, 64, 32), seed=2)
    np.testing.assert_array_equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(1, 1100, 2, 600, 24), (1, 1100, 1, 4096, 32)])
def test_noalloc_wide_keys(shape):
    # dk > 512: LDS-state path (600), and the scratch-tile path (4096), whose
    # 1024-token preparation chunk needs 67 MB and shrinks to fit the array
    got, want, _ = run_both(S(*shape), seed=3)
    np.testing.assert_array_equal(got, want)


@pytest.mark.gpu
def test_noalloc_packed_sequences():
    # packed sequences on the chunked path: 32 heads x 128 x 64 need 112 MB of
    # prepared blocks per 128-chunk window; in 64 MiB the windows shrink, and
    # the 3000- and 2100-token sequences carry their states across them
    import torch
    lengths = [3000, 0, 1500, 17, 2100]
    s = S(1, sum(lengths), 32, 128, 64, initial_state=False)
    inp = W.gated_deltanet2_inputs(s, seed=5)
    keys = KEYS[:-1]
    d = {k: to_dev(inp[k]) for k in keys}
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)).to("cuda")
    ref = xp.gated_deltanet2_fn(*(d[k] for k in keys), None, scale=s.scale, use_qk_l2norm_in_kernel=int(s.l2norm),
                                cu_seqlens=cu)
    out = torch.full_like(ref, float("nan"))
    descs = [xp._desc_from_tensor(d[k]) for k in keys] + [xp._desc_from_tensor(None), xp._desc_from_tensor(cu)]
    st, msg = _call_noalloc(descs, s, out.data_ptr(), torch.cuda.current_stream().cuda_stream, has_cu_seqlens=1)
    assert st == xp.XM_OK, msg
    launched = xp.last_launches()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), ref.cpu().numpy())
    assert any(k.startswith("Gdn2ChunkRecurKernel") for k in launched), launched


@pytest.mark.gpu
def test_noalloc_sequence_split():
    # few heads and 64 chunks: both entry points split the sequence (2 MB of scratch)
    got, want, launched = run_both(S(1, 1024, 2, 64, 32), seed=6)
    np.testing.assert_array_equal(got, want)
    assert any(k.startswith("Gdn2ChunkSplitKernel") for k in launched), launched


@pytest.mark.gpu
def test_noalloc_windows_where_the_split_exceeds_the_array():
    # 65536 tokens x 2 heads at 128 x 128: the split needs 0.2 GB of prepared
    # blocks, so the array steps the sequence in windows instead
    got, want, launched = run_both(S(1, 65536, 2, 128, 128), seed=7)
    assert not any(k.startswith("Gdn2ChunkSplitKernel") for k in launched), launched
    check("noalloc/windows_vs_split", got, want, TOL_GPU)


@pytest.mark.gpu
def test_noalloc_without_scratch_needs():
    # the sequential kernel (gdn2_path override) takes no scratch: the call
    # plans 0 bytes (test_capi_cpu checks the size), so the array is not used
    import torch
    s = S(1, 40, 2, 64, 16, initial_state=False)
    with xp.kernel_override("gdn2_path", 1):
        got, want, launched = run_both(s, seed=4)
    np.testing.assert_array_equal(got, want)
    assert launched and launched[0].startswith("Gdn2FusedKernel"), launched
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_noalloc_calls_on_two_streams_are_ordered():
    # A long call on one stream and, right after it with no host wait, another
    # call on a second stream: both use the one array, so the second waits for
    # the first's kernels (the device's event) before it overwrites it.  Each
    # output equals the allocating entry point's, bit for bit.
    import torch
    shapes = [S(4, 2100, 16, 128, 64), S(2, 1500, 8, 128, 64)]
    runs = []
    for i, s in enumerate(shapes):
        inp = W.gated_deltanet2_inputs(s, seed=20 + i)
        d = {k: to_dev(inp[k]) for k in KEYS}
        ref = xp.gated_deltanet2_fn(*(d[k] for k in KEYS), scale=s.scale, use_qk_l2norm_in_kernel=int(s.l2norm))
        runs.append((s, d, ref, torch.full_like(ref, float("nan"))))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for (s, d, _, out), st in zip(runs, streams):
        code, msg = _call_noalloc([xp._desc_from_tensor(d[k]) for k in KEYS], s, out.data_ptr(), st.cuda_stream)
        assert code == xp.XM_OK, msg
    torch.cuda.synchronize()
    for s, _, ref, out in runs:
        np.testing.assert_array_equal(out.cpu().numpy(), ref.cpu().numpy())


def test_noalloc_rejects_calls_beyond_the_array():
    # The carried state alone (64 heads x 512 x 512 fp32 = 64 MiB) leaves no
    # room for a window: rejected before anything is enqueued (no device use).
    s = S(1, 5000, 64, 512, 512)
    shapes = [(1, 5000, 64, 512)] * 2 + [(1, 5000, 64, 512)] + [(1, 5000, 64, 512)] * 2 + [(1, 5000, 64, 512)] + \
        [(1, 64, 512, 512)]
    descs = [xp._desc_from_shape(sh) for sh in shapes]
    st, msg = _call_noalloc(descs, s, xp._DUMMY.value, None)
    assert st == xp.XM_ERR_UNSUPPORTED
    assert "64 MiB" in msg and "xm_gated_deltanet2_forward" in msg
